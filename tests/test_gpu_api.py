"""GPU tests of the reference-facing API beyond the dynamic pipeline:
the kernel-level helpers of bsa_interface.py (attention fwd/bwd over given
tile lists, list transpose, selection, scores), the _run_bsa_dynamic adapter
(padding, shape cache, unpadding) and the error behaviour.  Edge cases the
reference guards: empty lists, fully padded key tiles, dense lists."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.cases import bf16, padded_case
from tests.test_gpu_parity import _tol, bits_equal, dev, host, say

pytestmark = pytest.mark.gpu


def _random_lists(rng, BH, M, width, empty_rows=(), full_rows=()):
    """Dense [BH, M, width] ascending tile lists padded with the sentinel M."""
    idx = np.full((BH, M, width), M, np.int64)
    lens = np.zeros((BH, M), np.int32)
    for bh in range(BH):
        for t in range(M):
            if (bh, t) in empty_rows:
                continue
            n = M if (bh, t) in full_rows else int(rng.integers(1, width + 1))
            n = min(n, width)
            idx[bh, t, :n] = np.sort(rng.choice(M, n, replace=False))
            lens[bh, t] = n
    return idx, lens


@pytest.mark.parametrize("D", [64, 128])
def test_kernel_level_fwd_bwd_vs_oracle(D):
    from prism_amd import bsa_interface as BI
    rng = np.random.default_rng(21)
    B, H, S = 1, 2, 2048
    M = S // 64
    say("kernel-level", D)
    q, k, v, do = (bf16(rng.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(4))
    idx, lens = _random_lists(rng, B * H, M, M, empty_rows={(0, 3), (1, 10)}, full_rows={(0, 5), (1, 0)})
    kv = (rng.random(S) > 0.15).astype(np.uint8)
    kv[7 * 64:8 * 64] = 0  # one fully padded key tile
    sm = 1 / math.sqrt(D)
    qt, kt, vt_, dot = (dev(x) for x in (q, k, v, do))
    bi = dev(idx.reshape(B, H, M, M))
    bl = dev(lens.reshape(B, H, M))
    o, lse = BI.attn_fwd_bsa_varlen(qt, kt, vt_, sm, bi, bl, 64, 64, kv_valid_mask=dev(kv))
    qs = np.arange(B * H * M, dtype=np.int64) * M
    tof = lambda a: O.bf16_bits_to_f32(a).reshape(B * H, S, D)
    o_ref, lse_ref = O.attn_fwd(tof(q), tof(k), tof(v), qs, lens.reshape(-1), idx.reshape(-1).astype(np.int32), kv, sm)
    og = O.bf16_bits_to_f32(host(o)).reshape(B * H, S, D)
    _tol(og, o_ref, "O")
    lg = host(lse).reshape(B * H, S)
    fin = np.isfinite(lse_ref)
    assert np.array_equal(np.isfinite(lg), fin)
    assert np.abs(lg[fin] - lse_ref[fin]).max() < 1e-3
    # empty lists: output 0 and lse -inf (the reference's all-masked guard)
    assert np.all(og[0, 3 * 64:4 * 64] == 0) and np.all(np.isneginf(lg[0, 3 * 64:4 * 64]))
    dq = torch.empty_like(qt); dk = torch.empty_like(kt); dv = torch.empty_like(vt_)
    BI.attn_bwd_bsa_varlen(dot, qt, kt, vt_, o, dq, dk, dv, sm, lse, bi, bl, 64, 64, kv_valid_mask=dev(kv))
    dq_r, dk_r, dv_r = O.attn_bwd(tof(q), tof(k), tof(v), og, tof(do), lse_ref, qs, lens.reshape(-1),
                                  idx.reshape(-1).astype(np.int32), kv, sm)
    for name, g, r in (("dQ", dq, dq_r), ("dK", dk, dk_r), ("dV", dv, dv_r)):
        _tol(O.bf16_bits_to_f32(host(g)).reshape(B * H, S, D), r, name)
    # fully padded key tile receives no gradient
    assert np.all(O.bf16_bits_to_f32(host(dk)).reshape(B * H, S, D)[:, 7 * 64:8 * 64] == 0)


def test_dense_lists_match_dense_attention():
    """All tiles listed and no mask: the block-sparse kernels are dense
    attention (torch fp32 reference on the CPU)."""
    from prism_amd import bsa_interface as BI
    rng = np.random.default_rng(5)
    B, H, S, D = 1, 2, 1024, 128
    M = S // 64
    q, k, v, do = (bf16(rng.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(4))
    idx = np.broadcast_to(np.arange(M), (B, H, M, M)).copy()
    lens = np.full((B, H, M), M, np.int32)
    sm = 1 / math.sqrt(D)
    qt, kt, vt_, dot = (dev(x) for x in (q, k, v, do))
    o, lse = BI.attn_fwd_bsa_varlen(qt, kt, vt_, sm, dev(idx), dev(lens))
    tq, tk, tv, tdo = (torch.from_numpy(O.bf16_bits_to_f32(x)).requires_grad_(True) for x in (q, k, v, do))
    ref = torch.softmax((tq @ tk.transpose(-1, -2)) * sm, -1) @ tv
    ref.backward(tdo.detach())
    _tol(O.bf16_bits_to_f32(host(o)), ref.detach().numpy().astype(np.float64), "O dense")
    dq = torch.empty_like(qt); dk = torch.empty_like(kt); dv = torch.empty_like(vt_)
    BI.attn_bwd_bsa_varlen(dot, qt, kt, vt_, o, dq, dk, dv, sm, lse, dev(idx), dev(lens))
    for name, g, r in (("dQ", dq, tq.grad), ("dK", dk, tk.grad), ("dV", dv, tv.grad)):
        _tol(O.bf16_bits_to_f32(host(g)), r.numpy().astype(np.float64), name + " dense")


def test_create_indices_k_from_indices_q_bitexact():
    from prism_amd import bsa_interface as BI
    rng = np.random.default_rng(9)
    B, H, M = 1, 3, 40
    idx, lens = _random_lists(rng, B * H, M, 12, empty_rows={(0, 1)})
    kc, kl = BI.create_indices_k_from_indices_q_varlen(dev(idx.reshape(B, H, M, 12)), M)
    qs = np.arange(B * H * M, dtype=np.int64) * 12
    ref_c, ref_l = O.transpose_lists(qs, lens.reshape(-1), idx.reshape(-1).astype(np.int32), B * H, M)
    kl = host(kl).reshape(-1)
    kc = host(kc).reshape(B * H * M, M)
    assert np.array_equal(kl, ref_l)
    for r in range(B * H * M):
        assert np.array_equal(kc[r, : kl[r]], ref_c[r, : kl[r]])
        assert np.all(kc[r, kl[r]:] == M)  # sentinel padding, as the reference's sort leaves it


@pytest.mark.parametrize("params", [(0.75, None), (None, 0.9), (0.95, 0.9)])
def test_selection_helpers_bitexact(params):
    from prism_amd import bsa_interface as BI
    sp, p = params
    rng = np.random.default_rng(13)
    N = 300
    s = (rng.standard_normal((1, 2, N, N)) * 3).astype(np.float32)
    sm = 1 / math.sqrt(128)
    if p is None:
        idx, lens = BI.get_select_indices_topk_from_score(dev(s), sp)
    elif sp is None:
        idx, lens = BI.get_select_indices_cdf_from_score(dev(s), p, sm)
    else:
        idx, lens = BI.get_select_indices_cdf_topk_from_score(dev(s), sp, p, sm)
    ref_sel, ref_n = O.select(s.reshape(-1, N), sp, p, sm)
    lens = host(lens).reshape(-1)
    idx = host(idx).reshape(2 * N, -1)
    assert np.array_equal(lens, ref_n)
    for r in range(2 * N):
        assert np.array_equal(idx[r, : lens[r]], ref_sel[r, : lens[r]])


def test_cal_score_bitexact():
    from prism_amd import bsa_interface as BI
    rng = np.random.default_rng(17)
    qc = rng.standard_normal((1, 2, 100, 128)).astype(np.float32)
    kc = rng.standard_normal((1, 2, 100, 128)).astype(np.float32)
    got = host(BI.cal_score(dev(qc), dev(kc))).reshape(2, 100, 100)
    assert bits_equal(got, O.block_scores(qc.reshape(2, 100, 128), kc.reshape(2, 100, 128), None))


def test_adapter_pads_caches_and_unpads():
    """_run_bsa_dynamic contract: an unpadded grid is padded to multiples of 8
    with a valid mask, audio norms padded with 0, output unpadded; in training
    the shape ids of one pass are reused by its recompute."""
    from prism_amd import DynamicBlockSparseAttention, flash_attn_bsa_3d_dynamic, valid_mask_for
    rng = np.random.default_rng(3)
    grid = (5, 12, 20)
    T, Hg, Wg = grid
    B, H, D = 1, 2, 64
    S = T * Hg * Wg
    q, k, v = (torch.from_numpy(rng.standard_normal((B, H, S, D)).astype(np.float32)).to("cuda").to(torch.bfloat16)
               for _ in range(3))
    norms = torch.from_numpy(rng.random(S).astype(np.float32)).to("cuda")
    att = DynamicBlockSparseAttention("ivpq", {"sparsity": 0.7, "cdf_threshold": 0.9})
    out = att(q, k, v, grid, norms)
    assert out.shape == (B, H, S, D) and out.dtype == torch.bfloat16
    gp = (8, 16, 24)
    pad = lambda t: torch.nn.functional.pad(t.view(B, H, T, Hg, Wg, D), (0, 0, 0, 4, 0, 4, 0, 3)).reshape(B, H, -1, D)
    npad = torch.nn.functional.pad(norms.view(T, Hg, Wg), (0, 4, 0, 4, 0, 3)).reshape(-1)
    ref, sid = flash_attn_bsa_3d_dynamic(pad(q), pad(k), pad(v), gp, method="ivpq", sparsity=0.7,
                                         cdf_threshold=0.9, audio_token_norms=npad,
                                         valid_mask=valid_mask_for(grid, "cuda"), return_shape_ids=True)
    ref = ref.view(B, H, *gp, D)[:, :, :T, :Hg, :Wg].reshape(B, H, S, D)
    assert torch.equal(out, ref)
    # shape cache: same pass id -> reuse; new pass -> recompute
    att.training = True
    att.advance_pass()
    att(q, k, v, grid, norms)
    first = att._dyn_shape_cache[2].clone()
    v2 = v * 0 + torch.randn_like(v)
    att(q, k, v2, grid, norms)
    assert torch.equal(att._dyn_shape_cache[2], first)
    att.advance_pass()
    att(q, k, v2, grid, norms)
    assert torch.equal(att._dyn_shape_cache[2], select_ids(v2, gp, pad, npad))


def _padder(B, H, grid, gp, D):
    (T, Hg, Wg), (Tp, Hp, Wp) = grid, gp
    def pad(t):
        if t.dim() == 1:
            return torch.nn.functional.pad(t.view(T, Hg, Wg), (0, Wp - Wg, 0, Hp - Hg, 0, Tp - T)).reshape(-1)
        return torch.nn.functional.pad(t.view(B, H, T, Hg, Wg, D),
                                       (0, 0, 0, Wp - Wg, 0, Hp - Hg, 0, Tp - T)).reshape(B, H, -1, D)
    return pad


@pytest.mark.parametrize("grid,D,dtype", [((5, 12, 20), 128, torch.bfloat16), ((8, 9, 16), 64, torch.float32),
                                          ((3, 8, 8), 128, torch.float32)])
def test_input_grid_box_kernels_equal_padding(grid, D, dtype):
    """Every kernel of the dynamic path that reads THW tensors, given the
    unpadded input grid, equals the same kernel over the zero-padded zone grid
    with the padding valid mask (wan_video_dit.py:342-400), bit for bit: zone
    statistics, audio statistics, gather + pooling + counts + rowdot, and the
    scatter back (with the slice of :429-431).  Also with a caller mask over
    the input grid."""
    from prism_amd import ops, select_zone_shapes, valid_mask_for
    from prism_amd.adapter import padded_grid
    rng = np.random.default_rng(31)
    B, H = 2, 3
    gp, _ = padded_grid(grid)
    S = int(np.prod(grid))
    say("box kernels", grid, D, dtype)
    pad = _padder(B, H, grid, gp, D)
    x = torch.from_numpy(rng.standard_normal((B, H, S, D)).astype(np.float32)).to("cuda").to(dtype)
    norms = torch.from_numpy(rng.random(S).astype(np.float32)).to("cuda").to(dtype)
    vpad = valid_mask_for(grid, "cuda")
    for own in (None, torch.from_numpy(rng.random(S) > 0.2).to("cuda")):
        vm_p = vpad if own is None else (vpad & pad(own.to(torch.uint8)).bool())
        p_b, av_b = ops.zone_stats(x, gp, own, box=grid)
        p_p, av_p = ops.zone_stats(pad(x), gp, vm_p)
        assert bits_equal(host(p_b), host(p_p)) and torch.equal(av_b, av_p)
        a_b, vh_b = ops.audio_zone_stats(norms, gp, own, box=grid)
        a_p, vh_p = ops.audio_zone_stats(pad(norms), gp, vm_p)
        assert bits_equal(host(a_b), host(a_p)) and bits_equal(host(vh_b), host(vh_p))
        sid = select_zone_shapes(pad(x), pad(norms), gp, "ivpq", valid_mask_thw=vm_p)
        lay_b, lay_p = ops.ZoneLayout(sid, gp, box=grid), ops.ZoneLayout(sid, gp)
        assert lay_b.padded and lay_b.S == lay_p.S and lay_b.N_b == lay_p.N_b
        g_b = ops.gather_pool(x, lay_b, own, rows=True, pool=True, counts=True)
        g_p = ops.gather_pool(pad(x), lay_p, vm_p, rows=True, pool=True, counts=True)
        for key in ("rows", "block_count", "tile_count", "valid_re"):
            assert torch.equal(g_b[key], g_p[key]), key
        assert bits_equal(host(g_b["block_mean"]), host(g_p["block_mean"]))
        d_b = ops.gather_pool(x, lay_b, None, rows=False, dot_with=g_p["rows"])["rowdot"]
        d_p = ops.gather_pool(pad(x), lay_p, None, rows=False, dot_with=g_p["rows"])["rowdot"]
        assert bits_equal(host(d_b), host(d_p))
        o_b = ops.scatter_rows(g_p["rows"], lay_b, dtype)
        o_p = ops.scatter_rows(g_p["rows"], lay_p, dtype)
        assert o_b.shape == (B, H, S, D)
        Tp, Hp, Wp = gp
        T, Hg, Wg = grid
        assert torch.equal(o_b, o_p.view(B, H, Tp, Hp, Wp, D)[:, :, :T, :Hg, :Wg].reshape(B, H, S, D))
        assert torch.equal(o_b, x.to(torch.bfloat16).to(dtype))  # gather then scatter is the identity
    with pytest.raises(ValueError, match="tokens"):
        ops.gather_pool(pad(x), ops.ZoneLayout(sid, gp, box=grid), None)


@pytest.mark.parametrize("grid,cpq", [((5, 12, 20), False), ((6, 16, 13), True)])
def test_input_grid_fwd_bwd_equal_padding(grid, cpq):
    """flash_attn_bsa_3d_dynamic over the unpadded grid (input_grid) equals the
    reference caller's flow (pad q, k, v and the audio norms, pass the valid
    mask, slice the output) bit for bit, output and the gradients of q, k, v."""
    from prism_amd import flash_attn_bsa_3d_dynamic, valid_mask_for
    from prism_amd.adapter import padded_grid
    rng = np.random.default_rng(37)
    B, H, D = 1, 2, 128
    gp, _ = padded_grid(grid)
    S = int(np.prod(grid))
    say("box fwd/bwd", grid, cpq)
    pad = _padder(B, H, grid, gp, D)
    base = [torch.from_numpy(rng.standard_normal((B, H, S, D)).astype(np.float32)).to("cuda").to(torch.bfloat16)
            for _ in range(3)]
    norms = torch.from_numpy(rng.random(S).astype(np.float32)).to("cuda").to(torch.bfloat16)
    do = torch.from_numpy(rng.standard_normal((B, H, S, D)).astype(np.float32)).to("cuda").to(torch.bfloat16)
    kw = dict(method="ivpq", sparsity=0.6, cdf_threshold=0.8, return_shape_ids=True, compute_padded_queries=cpq)
    q1, k1, v1 = (t.clone().requires_grad_(True) for t in base)
    out1, sid1 = flash_attn_bsa_3d_dynamic(q1, k1, v1, gp, audio_token_norms=norms, input_grid=grid, **kw)
    out1.backward(do)
    q2, k2, v2 = (t.clone().requires_grad_(True) for t in base)
    out2, sid2 = flash_attn_bsa_3d_dynamic(pad(q2), pad(k2), pad(v2), gp, audio_token_norms=pad(norms),
                                           valid_mask=valid_mask_for(grid, "cuda"), **kw)
    T, Hg, Wg = grid
    out2 = out2.view(B, H, *gp, D)[:, :, :T, :Hg, :Wg].reshape(B, H, S, D)
    out2.backward(do)
    assert torch.equal(sid1, sid2)
    assert torch.equal(out1, out2)
    for a, b in ((q1, q2), (k1, k2), (v1, v2)):
        assert torch.equal(a.grad, b.grad)


def select_ids(v, gp, pad, npad):
    from prism_amd import select_zone_shapes, valid_mask_for
    return select_zone_shapes(pad(v), npad, gp, "ivpq", valid_mask_thw=valid_mask_for((5, 12, 20), "cuda"))


def test_errors_match_reference():
    from prism_amd import flash_attn_bsa_3d_dynamic, select_zone_shapes
    x = torch.zeros((1, 1, 512, 64), device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        flash_attn_bsa_3d_dynamic(x, x, x, (8, 8, 8), method="ivpq", sparsity=None, cdf_threshold=None)
    with pytest.raises(AssertionError):
        flash_attn_bsa_3d_dynamic(x, x, x, (4, 8, 16), method="ivpq")
    with pytest.raises(ValueError):
        flash_attn_bsa_3d_dynamic(x, x, x, (8, 8, 8), method="nope")
    with pytest.raises(ValueError):
        select_zone_shapes(x, None, (8, 8, 8), "nope")
    with pytest.raises(ValueError, match="no CPU path"):
        flash_attn_bsa_3d_dynamic(x.cpu(), x.cpu(), x.cpu(), (8, 8, 8), method="ivpq")


def test_bad_shape_ids_raise():
    """Caller-supplied shape ids outside the 13-entry table, or of the wrong
    count or type, raise ValueError before any kernel but the (bounds-safe)
    zone layout reads them; good ids still work after a rejected call."""
    from prism_amd import flash_attn_bsa_3d_dynamic, ops
    x = torch.zeros((1, 1, 1024, 64), device="cuda", dtype=torch.bfloat16)
    grid = (8, 8, 16)  # two zones
    for bad in ([0, 13], [-1, 0], [0, 1, 2], [[0, 1]]):
        with pytest.raises(ValueError, match="shape_ids"):
            flash_attn_bsa_3d_dynamic(x, x, x, grid, method="ivpq", shape_ids=torch.tensor(bad, device="cuda"))
    with pytest.raises(ValueError, match="shape_ids"):
        flash_attn_bsa_3d_dynamic(x, x, x, grid, method="ivpq", shape_ids=torch.tensor([0.0, 1.0], device="cuda"))
    with pytest.raises(ValueError, match="shape_ids"):
        ops.rearrange_index(torch.tensor([3, 99], device="cuda"), grid)
    out, sid = flash_attn_bsa_3d_dynamic(x, x, x, grid, method="ivpq", shape_ids=torch.tensor([12, 0]),
                                         return_shape_ids=True)
    assert sid.tolist() == [12, 0] and out.shape == x.shape and bool(torch.isfinite(out).all())


def test_a2v_norms_adapter_batch0_dtype():
    from prism_amd import a2v_token_norms
    rng = np.random.default_rng(1)
    res = rng.standard_normal((2, 300, 512)).astype(np.float32)
    got = a2v_token_norms(torch.from_numpy(res).to("cuda").to(torch.bfloat16))
    assert got.dtype == torch.bfloat16 and got.shape == (300,)
    ref = O.a2v_norms(bf16(res[0]), True)
    assert np.array_equal(host(got), ref)


def test_padded_query_skip_leaves_valid_results_unchanged():
    """Fully padded query tiles are padding the caller slices away: skipping
    their attention leaves every valid output and every gradient at valid
    positions bit-identical when dO is 0 at padded positions."""
    from prism_amd import flash_attn_bsa_3d_dynamic
    c = padded_case(4, 1, 2, (11, 19, 13), 128, lowrank=True, audio_tokens=16)
    B, H, S, D = c["q"].shape
    valid = dev(c["valid"]).bool()
    rng = np.random.default_rng(8)
    do = torch.from_numpy(rng.standard_normal((B, H, S, D)).astype(np.float32)).to("cuda").to(torch.bfloat16)
    do = do * valid.view(1, 1, S, 1)
    res = []
    for compute_padded in (False, True):
        q, k, v = (dev(bf16(c[n])).requires_grad_(True) for n in ("q", "k", "v"))
        out = flash_attn_bsa_3d_dynamic(q, k, v, c["grid"], method="ivpq", sparsity=0.8, cdf_threshold=0.9,
                                        audio_token_norms=dev(c["norms"]), valid_mask=valid,
                                        compute_padded_queries=compute_padded)
        out.backward(do)
        res.append([host(t)[:, :, c["valid"].astype(bool)] for t in (out, q.grad, k.grad, v.grad)])
    for name, a, b in zip(("out", "dq", "dk", "dv"), *res):
        assert np.array_equal(a, b), name
