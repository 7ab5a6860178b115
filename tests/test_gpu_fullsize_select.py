"""Full-size checks of the selection side, and config 5 end to end.

  * zone statistics and shape ids of configs 2, 3 and 4 (inputs from
    bench.make_inputs) are bit-exact against the C oracle run on the same
    (zero-padded) inputs; the IVPQ decision margin of every zone (distance of
    the runner-up candidate minus the winner's, float64 from the kernels' g and
    rho, dynamic_block_shape.py:303-327) is reported, and wherever it exceeds
    float32 rounding the winner is the float64 argmin;
  * every score row of configs 2, 3, 4 and of config 5 at 5% and 25% is
    selected a second time by the reference's own torch op sequence (softmax /
    topk / cumsum / "cdf < p" + 1 / clamp, bsa_interface.py:235-304) in
    float32, on the GPU and with torch's CPU kernels, from the same fp32
    scores; the rows whose selected set differs from prism_select_tiles are
    counted, and each must have a weight tie at the cut or be decided
    within float32 cumsum rounding of p (|exact cumulative sum - p| <= 4e-6;
    at most 0.5% of the rows);
  * config 5 (the density sweep: config 4's tokens, seeded uniform shape ids
    passed as shape_ids=, top-k only) at 5%, 50% and 100% of the blocks:
    sampled selection rows bit-exact against the oracle, list structure,
    sampled O / LSE / dQ / dK / dV within tolerance of float64, repeated
    launches bit-identical; at 100% the whole output and all gradients are
    also compared with torch SDPA on the unpadded tensors (at k = N_b every
    query tile lists every key tile that holds a valid token, so the sparse
    path is dense attention);
  * config 1's selection parameters (top-8 blocks + p = 0.9, fp32, D = 64,
    padded grid, audio norms) end to end against the oracle.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle.torch_path import selection_agreement
from tests.test_gpu_fullsize import _attention, _list_structure, _selection_rows, _tol, say

pytestmark = pytest.mark.gpu
DEV = "cuda"
TILE = 64


def _host_bf16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _pad_thw(x: torch.Tensor, grid, gp) -> torch.Tensor:
    """[B,H,S,D] (or [S]) THW of grid -> zero-padded THW of the zone grid gp."""
    T, Hg, Wg = grid
    if x.dim() == 1:
        out = torch.zeros(gp, device=x.device, dtype=x.dtype)
        out[:T, :Hg, :Wg] = x.view(T, Hg, Wg)
        return out.reshape(-1)
    B, H, S, D = x.shape
    out = torch.zeros((B, H, *gp, D), device=x.device, dtype=x.dtype)
    out[:, :, :T, :Hg, :Wg] = x.view(B, H, T, Hg, Wg, D)
    return out.view(B, H, -1, D)


def _valid_thw(grid, gp) -> np.ndarray:
    v = np.zeros(gp, np.uint8)
    v[:grid[0], :grid[1], :grid[2]] = 1
    return v.reshape(-1)


def _ivpq_margins(g: np.ndarray, rho: np.ndarray, tau_128: float):
    """float64 IVPQ distances (dynamic_block_shape.py:303-327): per zone the
    argmin over the allowed candidates and the runner-up's distance minus the
    winner's."""
    shapes = np.log2(np.array(O.CANDIDATES, np.float64))           # [13, 3]
    is128 = np.prod(np.array(O.CANDIDATES), axis=1) == 128
    lr = (-2.0 / 3.0) * np.log2(g.astype(np.float64))              # [Nz, 3]
    ideal = lr + (6.0 - lr.sum(1, keepdims=True)) / 3.0
    dist = ((shapes[None] - ideal[:, None]) ** 2).sum(-1)            # [Nz, 13]
    dist[(rho[:, None] >= np.float32(tau_128)) & is128[None]] = np.inf
    order = np.argsort(dist, axis=1, kind="stable")
    best = order[:, 0]
    d0 = dist[np.arange(len(dist)), best]
    d1 = dist[np.arange(len(dist)), order[:, 1]]
    return best, d1 - d0


@pytest.mark.parametrize("cfg", ["c2", "c3", "c4"])
def test_zone_stats_and_shapes_fullsize_vs_oracle(cfg):
    import bench
    from prism_amd import a2v_token_norms, ops
    from prism_amd.adapter import padded_grid

    say("zones:", cfg)
    inp = bench.make_inputs(cfg)
    grid, D = inp["grid"], inp["D"]
    gp, _ = padded_grid(grid)
    with torch.no_grad():
        norms = a2v_token_norms(inp["res"])
        packed, av = ops.zone_stats(inp["v"], gp, None, grid)
        rho_raw, aniso = ops.zone_gradient(packed, av, D)
        abar, vhat = ops.audio_zone_stats(norms, gp, None, grid)
        g, rho, sid = ops.zone_shapes(rho_raw, aniso, abar, vhat, "ivpq", 0.5, 0.15, 1.0)
    torch.cuda.synchronize()
    valid = _valid_thw(grid, gp)
    say("zones: oracle statistics over", inp["H"], "heads")
    v_pad = _host_bf16(_pad_thw(inp["v"][:1], grid, gp))
    n_pad = _host_bf16(_pad_thw(norms, grid, gp))
    del inp
    ref_packed, ref_av = O.zone_stats(v_pad, gp, valid)
    del v_pad
    assert np.array_equal(packed.cpu().numpy().view(np.uint32), ref_packed.view(np.uint32))
    assert np.array_equal(av.cpu().numpy(), ref_av)
    ref_rho_raw, ref_aniso = O.zone_gradient(ref_packed, ref_av, D)
    ref_abar, ref_vhat = O.audio_zone_stats(n_pad, gp, valid)
    ref_g, ref_rho, ref_sid = O.zone_shapes(ref_rho_raw, ref_aniso, ref_abar, ref_vhat, "ivpq", 0.5, 0.15, 1.0)
    assert np.array_equal(g.cpu().numpy().view(np.uint32), ref_g.view(np.uint32))
    assert np.array_equal(rho.cpu().numpy().view(np.uint32), ref_rho.view(np.uint32))
    assert np.array_equal(sid.cpu().numpy(), ref_sid)
    # decision margins of the shape choice
    best, margin = _ivpq_margins(ref_g, ref_rho, 0.15)
    decided = margin > 1e-5
    assert np.array_equal(best[decided], ref_sid[decided])
    counts = np.bincount(ref_sid, minlength=13)
    say("zones:", cfg, "Nz", len(ref_sid), "shape histogram", counts.tolist(), "min argmin margin",
        float(margin.min()), "zones with margin < 1e-3:", int((margin < 1e-3).sum()),
        "< 1e-5:", int((~decided).sum()))


# How far from p a row's exact cumulative sum may lie when torch's float32
# sequence and the exact fixed-point rule decide it differently.  torch's
# cumsum adds c float32 weights (c < 1,000 at the crossing of every config
# here) to a running sum below 1, each addition rounding by at most 2^-25, so
# the accumulated error is a walk of c roughly uniform steps of standard
# deviation 2^-25 / sqrt(3): about 5.4e-7 at c = 1,000; torch's softmax adds
# a common relative error of a few 2^-24 to every weight.  4e-6 is seven
# standard deviations of that walk.  A threshold or rounding mistake of
# 1e-5 or more in the selection would put differing rows beyond it.
TORCH_SEQ_BOUND = 4e-6
# at most this fraction of the rows may decide differently without a weight
# tie at the cut (config 4: 0.15%); tied rows differ by torch.topk's
# unspecified tie order (torch's CPU kernel breaks ties differently from its
# GPU kernel and from the lower-index rule here)
TORCH_SEQ_MAX_FRAC = 5e-3
TORCH_SEQ_CASES = ["c2", "c3", "c4", "c5_0.05", "c5_0.25"]


def _selection_inputs(case):
    """Scores and selection parameters exactly as the benchmark runs `case`
    (c2-c4: bench.make_inputs with the config's shapes and top-k + p; c5_d:
    config 4's tokens, seed-5 uniform shape ids passed as shape_ids=, top-k
    with k = round(d N_b), as `bench.py --sweep`)."""
    import bench
    from prism_amd import a2v_token_norms, ops, plan_dynamic
    from prism_amd.adapter import padded_grid
    from prism_amd.dynamic_block_shape import ALL_CANDIDATE_SHAPES, _gradient_and_shapes
    from tests.test_gpu_fullsize import _sparsity

    cfg = case.split("_")[0]
    inp = bench.make_inputs("c4" if cfg == "c5" else cfg)
    grid, D = inp["grid"], inp["D"]
    gp, _ = padded_grid(grid)
    with torch.no_grad():
        if cfg == "c5":
            Nz = (gp[0] // 8) * (gp[1] // 8) * (gp[2] // 8)
            gen = torch.Generator(device=DEV).manual_seed(5)
            sid = torch.randint(0, len(ALL_CANDIDATE_SHAPES), (Nz,), generator=gen, device=DEV, dtype=torch.int64)
            N_b = ops.ZoneLayout(sid, gp, grid).N_b
            kk = max(1, min(N_b, round(float(case.split("_")[1]) * N_b)))
            sp, cdf, norms = 1.0 - (kk + 0.5) / N_b, None, None
        else:
            norms = a2v_token_norms(inp["res"])
            sid = _gradient_and_shapes(inp["v"], norms, gp, "ivpq", 0.5, 0.15, 1.0, None, grid)[2]
            N_b = ops.ZoneLayout(sid, gp, grid).N_b
            sp, cdf = _sparsity(inp, N_b)
        plan = plan_dynamic(inp["q"], inp["k"], inp["v"], gp, method="ivpq", sparsity=sp, cdf_threshold=cdf,
                            audio_token_norms=norms, input_grid=grid, keep_scores=True,
                            shape_ids=sid if cfg == "c5" else None)
    return plan, N_b, sp, cdf, 1 / math.sqrt(D)


@pytest.mark.parametrize("case", TORCH_SEQ_CASES)
def test_selection_vs_reference_torch_sequence_fullsize(case):
    """Every score row selected a second time by the reference's op sequence
    in float32, on the GPU and with torch's CPU kernels, from the same scores;
    the rows whose set differs from prism_select_tiles are counted, and each
    is a weight tie at the cut or lies within TORCH_SEQ_BOUND of p (at most
    TORCH_SEQ_MAX_FRAC of the rows are of the second kind)."""
    from prism_amd import ops

    say("torch sequence:", case)
    plan, N_b, sp, cdf, sm = _selection_inputs(case)
    with torch.no_grad():
        scores = plan.scores.view(-1, N_b)
        ours = ops.select_tiles(scores, sp, cdf, sm, plan.lay.block_first_tile, plan.tile_count, want_blocks=True)
    R = scores.shape[0]
    counts = selection_agreement(scores, ours["sel_blocks"], ours["nsel"], sp, cdf, sm)
    for name, c in counts.items():
        n_diff, n_tie, worst = c["rows_differing"], c["of_them_tied"], c["max_untied_margin"]
        say("torch sequence:", case, name, "rows", R, "N_b", N_b, "rows whose set differs", n_diff,
            f"({n_diff / R:.2e})", "of them with a boundary tie", n_tie, "largest |cdf - p| of an untied differing row",
            worst)
        assert worst <= TORCH_SEQ_BOUND, (case, name, "row differs at margin", worst, TORCH_SEQ_BOUND)
        assert n_diff - n_tie <= TORCH_SEQ_MAX_FRAC * R, (case, name, n_diff, n_tie, R)
    del plan, scores, ours
    torch.cuda.empty_cache()


SWEEP = [0.05, 0.5, 1.0]


@pytest.mark.parametrize("density", SWEEP)
def test_c5_density_sweep_fullsize(density):
    """Config 5 exactly as `bench.py --sweep` runs it (seed-5 uniform shape
    ids, sparsity 1 - (k + 0.5) / N_b, k = round(d N_b); s = 0 at k = N_b)."""
    import bench
    from prism_amd import flash_attn_bsa_3d_dynamic, ops, plan_dynamic
    from prism_amd.adapter import padded_grid
    from prism_amd.dynamic_block_shape import ALL_CANDIDATE_SHAPES

    say("c5: density", density)
    inp = bench.make_inputs("c4")
    B, H, D, grid = inp["B"], inp["H"], inp["D"], inp["grid"]
    gp, _ = padded_grid(grid)
    BH, sm = B * H, 1 / math.sqrt(D)
    Nz = (gp[0] // 8) * (gp[1] // 8) * (gp[2] // 8)
    gen = torch.Generator(device=DEV).manual_seed(5)
    sid = torch.randint(0, len(ALL_CANDIDATE_SHAPES), (Nz,), generator=gen, device=DEV, dtype=torch.int64)
    N_b = ops.ZoneLayout(sid, gp, grid).N_b
    kk = max(1, min(N_b, round(density * N_b)))
    sp = 0.0 if kk == N_b else 1.0 - (kk + 0.5) / N_b
    assert int((1 - sp) * N_b) == kk
    with torch.no_grad():
        plan = plan_dynamic(inp["q"], inp["k"], inp["v"], gp, method="ivpq", sparsity=sp, cdf_threshold=None,
                            shape_ids=sid, input_grid=grid, keep_scores=True)
    lay, Nt = plan.lay, plan.lay.Nt
    tiles, ntiles, tcap = plan.sel["tiles"], plan.sel["ntiles"], plan.sel["tcap"]
    rng = np.random.default_rng(8)
    _, kbt, nb, _ = O.tile_maps(sid.cpu().numpy())
    assert nb == N_b
    _selection_rows(rng, plan.scores.view(BH, N_b, N_b), tiles, ntiles, tcap, sp, None, sm, kbt, Nt,
                    plan.tile_count.cpu().numpy())
    _list_structure(tiles, ntiles, tcap, Nt, N_b, BH, lay.block_id_of_tile, plan.qstart, plan.qlen,
                    plan.tile_count)
    if kk == N_b:
        # every query tile with a valid token lists every key tile with one
        n_valid_k = int((plan.tile_count > 0).sum())
        q_live = plan.tile_count.repeat(BH) > 0
        assert bool((plan.qlen[q_live] == n_valid_k).all())
    plan.scores = None

    say("c5: forward")
    o, lse = ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qunion, sm, plan.qpair, plan.qorder)
    o2, lse2 = ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qunion, sm, plan.qpair, plan.qorder)
    assert torch.equal(o.view(torch.int16), o2.view(torch.int16))
    assert torch.equal(lse.view(torch.int32), lse2.view(torch.int32))
    del o2, lse2
    say("c5: backward")
    gd = ops.gather_pool(inp["do"], lay, None, rows=True, dot_with=o)
    do_re, delta = gd["rows"], gd["rowdot"]
    klists = ops.transpose_lists(plan.qstart, plan.qlen, plan.qcols, BH, Nt)
    kpair = ops.pair_tiles(*klists, Nt)
    kunion = ops.pair_union(*klists, Nt, pairmap=kpair)
    korder = ops.pair_order(kunion[1], 32)
    m2 = ops.lse_to_m2(lse)
    dq, dk, dv = ops.bsa_bwd(plan.q_re, plan.k_re, plan.v_re, do_re, m2, delta, plan.kv_valid, plan.tmasks,
                             plan.qunion, kunion, sm, plan.qpair, kpair, plan.qorder, korder)
    again = ops.bsa_bwd(plan.q_re, plan.k_re, plan.v_re, do_re, m2, delta, plan.kv_valid, plan.tmasks,
                        plan.qunion, kunion, sm, plan.qpair, kpair, plan.qorder, korder)
    for g_, g2 in zip((dq, dk, dv), again):
        assert torch.equal(g_.view(torch.int16), g2.view(torch.int16))
    del again
    torch.cuda.synchronize()
    nq, nk = (3, 2) if kk == N_b else (6, 3)
    _attention(rng, plan.q_re, plan.k_re, plan.v_re, plan.kv_valid, o, lse, do_re, delta, dq, dk, dv, plan.qstart,
               plan.qlen, plan.qcols, klists, BH, Nt, D, sm, nq=nq, nk=nk)
    del plan, o, lse, dq, dk, dv, do_re, gd, klists, kunion, m2, delta
    torch.cuda.empty_cache()

    if kk == N_b:
        say("c5: 100% density vs torch SDPA (whole tensors)")
        q, k, v = (inp[n].clone().requires_grad_(True) for n in ("q", "k", "v"))
        out = flash_attn_bsa_3d_dynamic(q, k, v, gp, method="ivpq", sparsity=sp, cdf_threshold=None, shape_ids=sid,
                                        input_grid=grid)
        out.backward(inp["do"])
        qd, kd, vd = (inp[n].clone().requires_grad_(True) for n in ("q", "k", "v"))
        ref = torch.nn.functional.scaled_dot_product_attention(qd, kd, vd)
        ref.backward(inp["do"])
        torch.cuda.synchronize()
        for name, a, b in (("O", out, ref), ("dQ", q.grad, qd.grad), ("dK", k.grad, kd.grad), ("dV", v.grad, vd.grad)):
            a64, b64 = a.detach().double(), b.detach().double()
            err = (a64 - b64).abs()
            rel = float((a64 - b64).norm() / b64.norm())
            say("c5 vs SDPA", name, "max-abs", float(err.max()), "mean-abs", float(err.mean()), "rel", rel)
            assert float(err.max()) <= 2e-2 and float(err.mean()) <= 2e-3 and rel <= 2e-2, name
        del q, k, v, out, qd, kd, vd, ref
    del inp
    torch.cuda.empty_cache()


def test_c1_parameters_topk8_p09():
    """Config 1's selection parameters: top-8 blocks plus p = 0.9 through
    flash_attn_bsa_3d_dynamic (sparsity 1 - (8 + 0.5) / N_b with the shape
    ids passed in, as the config prescribes; fp32 inputs, D = 64, grid
    4x16x16 padded to 8x16x16, 64 audio tokens), forward and backward vs the
    oracle on its own selection."""
    from prism_amd import flash_attn_bsa_3d_dynamic
    from tests.cases import bf16, padded_case
    from tests.test_gpu_parity import dev

    c = padded_case(0, 1, 4, (4, 16, 16), 64, audio_tokens=64)
    B, H, S, D = c["q"].shape
    grid, valid = c["grid"], c["valid"]
    sid = O.select_zone_shapes(c["v"], c["norms"], grid, "ivpq", valid=valid)
    _, _, N_b, _ = O.tile_maps(sid)
    sp = 1.0 - (8 + 0.5) / N_b
    assert int((1 - sp) * N_b) == 8
    sm = 1 / math.sqrt(D)
    ref = O.select_pipeline(c["q"], c["k"], c["v"], grid, method="ivpq", sparsity=sp, cdf_threshold_p=0.9,
                            audio_norms=c["norms"], valid=valid, shape_ids=sid, skip_padded_queries=False)
    assert int(ref["nsel"].min()) >= 8
    src, inv = O.rearrange_index(sid, grid)
    tof = lambda a: O.bf16_bits_to_f32(bf16(a))[:, :, src].reshape(B * H, S, D)
    qf, kf, vf = tof(c["q"]), tof(c["k"]), tof(c["v"])
    o_ref, lse_ref = O.attn_fwd(qf, kf, vf, ref["qstart"], ref["qlen"], ref["qcols"], valid[src], sm)
    q, k, v = (dev(c[n]).requires_grad_(True) for n in ("q", "k", "v"))
    out, got_sid = flash_attn_bsa_3d_dynamic(q, k, v, grid, method="ivpq", sparsity=sp, cdf_threshold=0.9,
                                             audio_token_norms=dev(c["norms"]), valid_mask=dev(valid).bool(),
                                             shape_ids=dev(sid), return_shape_ids=True)
    assert out.dtype == torch.float32
    assert np.array_equal(got_sid.cpu().numpy(), sid)
    _tol(out.detach().cpu().numpy().reshape(B * H, S, D), o_ref[:, inv], "C1 O")
    rng = np.random.default_rng(12)
    do = O.bf16_bits_to_f32(bf16(rng.standard_normal((B, H, S, D)).astype(np.float32)))
    out.backward(torch.from_numpy(do).to(DEV))
    o_bf = O.bf16_bits_to_f32(bf16(o_ref.astype(np.float32)))
    grads = O.attn_bwd(qf, kf, vf, o_bf, do.reshape(B * H, S, D)[:, src], lse_ref, ref["qstart"], ref["qlen"],
                       ref["qcols"], valid[src], sm)
    for name, t, r in zip(("dQ", "dK", "dV"), (q, k, v), grads):
        _tol(t.grad.cpu().numpy().reshape(B * H, S, D), r[:, inv], "C1 " + name)
