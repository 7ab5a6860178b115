"""Parity at the full sizes of the BASELINE GPU configs:
  c4  2K:    B=1, H=5,  D=128, input grid 21x90x160, top-48 + p = 0.9
  c3  1080p: B=1, H=24, D=128, input grid 21x68x120, top-32 + p = 0.9
  c2  720p:  B=1, H=24, D=128, input grid 21x45x80,  sparsity 0.75
(inputs from bench.make_inputs, the benchmark's own generator), through the
dynamic-shape path (flash_attn_bsa_3d_dynamic's plan and kernels), for c3
and c4 the uniform 4x4x4-chunk path (flash_attn_bsa_3d), and at c4 the v2a
bridge cross-attention (flash_attn_bsa_cross, audio queries over video keys).

The whole plan and the attention kernels run at full size; the float64
oracle checks what it finishes in seconds:
  * the tile lists of sampled score rows are bit-exact against the oracle's
    selection and tile expansion of the same fp32 scores;
  * every list is strictly ascending inside [0, Nt), and every query tile's
    list is the list of its block row (empty for tiles without a valid
    query token);
  * O and LSE of sampled query tiles, and their dQ (a query tile's dQ
    depends on its own list only), are within the north-star tolerance of
    the float64 oracle;
  * dK and dV of sampled key tiles sum over every query tile that lists
    them; they are checked against float64 sums over those query tiles with
    each query row's LSE taken from the kernels (the LSE itself is checked on
    the sampled query rows) and delta = rowsum(O dO) recomputed in float64
    from the stored O and dO (the kernels' delta is compared with it);
  * two forward launches give bit-identical O and LSE, two backward
    launches bit-identical dQ, dK and dV.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
TILE = 64


def say(*a):
    print(*a, flush=True)


def _tol(got, ref, what, rel_bound=1e-2):
    """max-abs 2e-2, mean-abs 2e-3 (bf16 vs float64); plus
    a relative bound ||got - ref|| / ||ref|| <= 1e-2 (Frobenius), which
    catches a scaled result where the values are small (at long lists |O| and
    |dQ| average ~6e-3, below the absolute bounds)."""
    diff = got.astype(np.float64) - ref
    err = np.abs(diff)
    mx, mean = float(err.max()), float(err.mean())
    ref_norm = float(np.linalg.norm(ref))
    rel = float(np.linalg.norm(diff)) / ref_norm if ref_norm > 0 else float(np.linalg.norm(diff))
    say(what, "max-abs", mx, "mean-abs", mean, "rel", rel, "||ref||", ref_norm)
    assert mx <= 2e-2 and mean <= 2e-3, (what, mx, mean)
    assert rel <= rel_bound, (what, "relative error", rel, "||ref||", ref_norm)


def _rows(t, bh, first, count):
    """Rows [first, first + count) of head bh of a [B, H, S, D] tile-order tensor, as float32 numpy."""
    return t.view(-1, t.shape[-2], t.shape[-1])[bh, first:first + count].float().cpu().numpy()


def _selection_rows(rng, scores, tiles, ntiles, tcap, sp, cdf, sm, kbt, Nt, tile_count):
    """Tile lists of 48 sampled score rows vs the oracle's selection and tile
    expansion of the same fp32 scores (bit-exact)."""
    say("fullsize: selection of sampled rows")
    R, N = scores.shape[0] * scores.shape[1], scores.shape[2]
    rows = np.sort(rng.choice(R, 48, replace=False))
    ridx = torch.as_tensor(rows, device=DEV)
    sel, nsel = O.select(scores.reshape(R, N)[ridx].cpu().numpy(), sp, cdf, sm)
    ref_tiles, ref_n = O.expand_tiles(sel, nsel, kbt, Nt, tile_count)
    got_n = ntiles.view(-1)[ridx].cpu().numpy()
    got_t = tiles.view(R, tcap)[ridx].cpu().numpy()
    assert np.array_equal(got_n, ref_n)
    for i in range(len(rows)):
        assert np.array_equal(got_t[i, : got_n[i]], ref_tiles[i, : ref_n[i]]), rows[i]


def _list_structure(tiles, ntiles, tcap, Ntk, N_b, BH, block_id_of_tile, qstart, qlen, q_tile_count):
    """Every list strictly ascending in [0, Ntk); each query tile carries its
    block row's list, empty where the tile holds no valid query token."""
    say("fullsize: list structure")
    t2 = tiles.view(-1, tcap)
    live = torch.arange(tcap, device=DEV)[None, :] < ntiles.view(-1, 1)
    assert bool(((t2 >= 0) & (t2 < Ntk) | ~live).all())
    assert bool(((t2[:, 1:] > t2[:, :-1]) | ~live[:, 1:]).all())
    del live
    brow = (torch.arange(BH, device=DEV)[:, None] * N_b + block_id_of_tile.long()[None, :]).reshape(-1)
    assert torch.equal(qstart, brow * tcap)
    want_len = torch.where(q_tile_count.repeat(BH) == 0, 0, ntiles.view(-1)[brow])
    assert torch.equal(qlen.long(), want_len.long())
    say("fullsize: kept tile pairs", int(qlen.sum()))


def _attention(rng, q_re, k_re, v_re, kv_valid, o, lse, do_re, delta, dq, dk, dv, qstart, qlen, qcols, klists,
               BH, Nt, D, sm, nq=6, nk=3):
    """O, LSE, dQ of nq sampled query tiles vs the float64 oracle; dK, dV of
    nk sampled key tiles vs float64 sums over the query tiles that list them
    (the last of each is the tile with the longest list)."""
    kv = kv_valid.cpu().numpy().astype(bool)
    lse_h = lse.view(BH, -1)
    delta_h = delta.view(BH, -1)
    qlen_h = qlen.cpu().numpy()
    qstart_h = qstart.cpu().numpy()
    cand = np.nonzero(qlen_h > 0)[0]
    pick = list(rng.choice(cand, nq - 1, replace=False)) + [int(cand[np.argmax(qlen_h[cand])])]
    for r in pick:
        bh, t = divmod(int(r), Nt)
        n = int(qlen_h[r])
        say("fullsize: query tile", bh, t, "keys", n)
        cols = qcols[int(qstart_h[r]): int(qstart_h[r]) + n].cpu().numpy()
        keys = O._row_keys(cols, 0, n)
        kidx = torch.as_tensor(keys, device=DEV)
        # tile 0 of the oracle's sequence holds the queries, tiles 1..n the listed keys
        Sx = TILE * (n + 1)
        qx, kx, vx, dox = (np.zeros((1, Sx, D), np.float32) for _ in range(4))
        qx[0, :TILE] = _rows(q_re, bh, t * TILE, TILE)
        dox[0, :TILE] = _rows(do_re, bh, t * TILE, TILE)
        kx[0, TILE:] = k_re.view(BH, -1, D)[bh][kidx].float().cpu().numpy()
        vx[0, TILE:] = v_re.view(BH, -1, D)[bh][kidx].float().cpu().numpy()
        kvx = np.zeros(Sx, np.uint8)
        kvx[TILE:] = kv[keys]
        st = np.zeros(n + 1, np.int64)
        ln = np.zeros(n + 1, np.int32)
        ln[0] = n
        lc = np.arange(1, n + 1, dtype=np.int32)
        o_ref, lse_ref = O.attn_fwd(qx, kx, vx, st, ln, lc, kvx, sm)
        _tol(_rows(o, bh, t * TILE, TILE), o_ref[0, :TILE], "O")
        lg = lse_h[bh, t * TILE:(t + 1) * TILE].cpu().numpy()
        fin = np.isfinite(lse_ref[0, :TILE])
        assert np.array_equal(np.isfinite(lg), fin)
        if fin.any():
            assert np.abs(lg[fin] - lse_ref[0, :TILE][fin]).max() < 1e-3
        dq_ref = O.attn_bwd(qx, kx, vx, o_ref, dox, lse_ref, st, ln, lc, kvx, sm)[0]
        _tol(_rows(dq, bh, t * TILE, TILE), dq_ref[0, :TILE], "dQ")
    kstart, klen, kcols = (x.cpu().numpy() for x in klists)
    kcand = np.nonzero(klen > 0)[0]
    kpick = list(rng.choice(kcand, nk - 1, replace=False)) + [int(kcand[np.argmax(klen[kcand])])]
    for r in kpick:
        bh, j = divmod(int(r), klen.size // BH)
        n = int(klen[r])
        say("fullsize: key tile", bh, j, "query tiles", n)
        qt = kcols[int(kstart[r]): int(kstart[r]) + n].astype(np.int64)
        qi = torch.as_tensor((qt[:, None] * TILE + np.arange(TILE)[None, :]).reshape(-1), device=DEV)
        Qs = q_re.view(BH, -1, D)[bh][qi].double().cpu().numpy()
        dOs = do_re.view(BH, -1, D)[bh][qi].double().cpu().numpy()
        Ls = lse_h[bh][qi].double().cpu().numpy()
        # delta = rowsum(O dO) in float64 from the stored bf16 O and dO rows
        # (not the kernels' delta, which is only compared with it)
        Os = o.view(BH, -1, D)[bh][qi].double().cpu().numpy()
        prod = Os * dOs
        dls = prod.sum(1)
        dk_delta = delta_h[bh][qi].double().cpu().numpy()
        # float32 sum of D products: |error| <= D 2^-24 sum |o do|
        assert (np.abs(dk_delta - dls) <= D * 2.0 ** -24 * np.abs(prod).sum(1) + 1e-30).all(), "delta"
        Kj = _rows(k_re, bh, j * TILE, TILE).astype(np.float64)
        Vj = _rows(v_re, bh, j * TILE, TILE).astype(np.float64)
        s = Qs @ Kj.T * sm
        s[:, ~kv[j * TILE:(j + 1) * TILE]] = -np.inf
        p = np.zeros_like(s)
        ok = np.isfinite(Ls)
        p[ok] = np.exp(s[ok] - Ls[ok, None])
        ds = p * (dOs @ Vj.T - dls[:, None])
        _tol(_rows(dk, bh, j * TILE, TILE), ds.T @ Qs * sm, "dK")
        _tol(_rows(dv, bh, j * TILE, TILE), p.T @ dOs, "dV")


def _sparsity(inp, N_b):
    """The benchmark's selection parameters: top-k exactly via sparsity
    1 - (k + 0.5) / N_b plus the threshold, or the config's sparsity."""
    if inp["sp_only"] is not None:
        return inp["sp_only"], None
    return 1.0 - (inp["topk"] + 0.5) / N_b, inp["cdf"]


@pytest.mark.parametrize("cfg", ["c2", "c3", "c4", "c4_d64"])
def test_full_size(cfg):
    """c4_d64: config 4's tokens and lists with head_dim 64 (config 1's head
    size; the first 64 channels of config 4's inputs), for the D = 64
    kernels at full size."""
    import bench
    from prism_amd import a2v_token_norms, ops, plan_dynamic
    from prism_amd.adapter import padded_grid
    from prism_amd.dynamic_block_shape import _gradient_and_shapes

    say("fullsize:", cfg, "inputs")
    inp = bench.make_inputs(cfg.split("_")[0])
    if cfg.endswith("_d64"):
        for name in ("q", "k", "v", "do"):
            inp[name] = inp[name][..., :64].contiguous()
        inp["D"] = 64
    B, H, D, grid = inp["B"], inp["H"], inp["D"], inp["grid"]
    gp, _ = padded_grid(grid)
    BH, sm = B * H, 1 / math.sqrt(D)
    say("fullsize: plan")
    norms = a2v_token_norms(inp["res"])
    with torch.no_grad():
        sid = _gradient_and_shapes(inp["v"], norms, gp, "ivpq", 0.5, 0.15, 1.0, None, grid)[2]
        N_b = ops.ZoneLayout(sid, gp, grid).N_b
        sp, cdf = _sparsity(inp, N_b)
        plan = plan_dynamic(inp["q"], inp["k"], inp["v"], gp, method="ivpq", sparsity=sp, cdf_threshold=cdf,
                            audio_token_norms=norms, input_grid=grid, keep_scores=True)
    lay, Nt = plan.lay, plan.lay.Nt
    assert lay.N_b == N_b and plan.S == gp[0] * gp[1] * gp[2]
    tiles, ntiles, tcap = plan.sel["tiles"], plan.sel["ntiles"], plan.sel["tcap"]
    rng = np.random.default_rng(4)
    _, kbt, nb, _ = O.tile_maps(lay.shape_ids.cpu().numpy())
    assert nb == N_b
    _selection_rows(rng, plan.scores.view(BH, N_b, N_b), tiles, ntiles, tcap, sp, cdf, sm, kbt, Nt,
                    plan.tile_count.cpu().numpy())
    _list_structure(tiles, ntiles, tcap, Nt, N_b, BH, lay.block_id_of_tile, plan.qstart, plan.qlen,
                    plan.tile_count)

    say("fullsize: forward")
    o, lse = ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qunion, sm, plan.qpair, plan.qorder)
    o2, lse2 = ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qunion, sm, plan.qpair, plan.qorder)
    assert torch.equal(o.view(torch.int16), o2.view(torch.int16))
    assert torch.equal(lse.view(torch.int32), lse2.view(torch.int32))
    del o2, lse2
    say("fullsize: backward")
    gd = ops.gather_pool(inp["do"], lay, None, rows=True, dot_with=o)
    do_re, delta = gd["rows"], gd["rowdot"]
    klists = ops.transpose_lists(plan.qstart, plan.qlen, plan.qcols, BH, Nt)
    kpair = ops.pair_tiles(*klists, Nt)
    kunion = ops.pair_union(*klists, Nt, pairmap=kpair)
    korder = ops.pair_order(kunion[1], 32)
    m2 = ops.lse_to_m2(lse)
    dq, dk, dv = ops.bsa_bwd(plan.q_re, plan.k_re, plan.v_re, do_re, m2, delta, plan.kv_valid, plan.tmasks,
                             plan.qunion, kunion, sm, plan.qpair, kpair, plan.qorder, korder)
    # a second backward launch gives the same bits (no atomics, fixed orders)
    again = ops.bsa_bwd(plan.q_re, plan.k_re, plan.v_re, do_re, m2, delta, plan.kv_valid, plan.tmasks,
                        plan.qunion, kunion, sm, plan.qpair, kpair, plan.qorder, korder)
    for g, g2 in zip((dq, dk, dv), again):
        assert torch.equal(g.view(torch.int16), g2.view(torch.int16))
    del again
    torch.cuda.synchronize()
    _attention(rng, plan.q_re, plan.k_re, plan.v_re, plan.kv_valid, o, lse, do_re, delta, dq, dk, dv, plan.qstart,
               plan.qlen, plan.qcols, klists, BH, Nt, D, sm)
    del plan, o, lse, dq, dk, dv, do_re, gd, inp
    torch.cuda.empty_cache()


@pytest.mark.parametrize("cfg", ["c3", "c4"])
def test_full_size_uniform(cfg):
    """The uniform path as benchmarked (`bench.py --path uniform`): 4x4x4
    chunks on the grid padded to whole chunks, flash_attn_bsa_3d's plan and
    kernels."""
    import bench
    from prism_amd import ops
    from prism_amd.uniform_block_attention import plan_chunked

    say("fullsize uniform:", cfg, "inputs")
    inp = bench.make_inputs(cfg)
    B, H, D, grid = inp["B"], inp["H"], inp["D"], inp["grid"]
    BH, sm = B * H, 1 / math.sqrt(D)
    lay = ops.ChunkLayout(grid, (4, 4, 4), DEV)
    sp, cdf = _sparsity(inp, lay.N_b)
    say("fullsize uniform: plan")
    plan = plan_chunked(inp["q"], inp["k"], inp["v"], lay, lay, sparsity=sp, cdf_threshold=cdf, sm_scale=sm,
                        keep_scores=True)
    Nt, N_b = lay.Nt, lay.N_b
    assert plan.kv_valid is not None  # the padded grid has padding rows
    tile_count = plan.kv_valid.view(-1, TILE).sum(1, dtype=torch.int32)
    tiles, ntiles, tcap = plan.sel["tiles"], plan.sel["ntiles"], plan.sel["tcap"]
    rng = np.random.default_rng(5)
    kbt = O.chunk_kblock_tiles(N_b, lay.csz, Nt)
    _selection_rows(rng, plan.scores.view(BH, N_b, N_b), tiles, ntiles, tcap, sp, cdf, sm, kbt, Nt,
                    tile_count.cpu().numpy())
    _list_structure(tiles, ntiles, tcap, Nt, N_b, BH, lay.block_id_of_tile, plan.qstart, plan.qlen, tile_count)

    say("fullsize uniform: forward")
    o, lse = ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qunion, sm, plan.qpair, plan.qorder)
    say("fullsize uniform: backward")
    gd = ops.chunk_gather_pool(inp["do"], lay, None, rows=True, dot_with=o)
    do_re, delta = gd["rows"], gd["rowdot"]
    kunion = plan.key_lists()
    m2 = ops.lse_to_m2(lse)
    dq, dk, dv = ops.bsa_bwd(plan.q_re, plan.k_re, plan.v_re, do_re, m2, delta, plan.kv_valid, plan.tmasks,
                             plan.qunion, kunion, sm, plan.qpair, plan.kpair, plan.qorder, plan.korder)
    torch.cuda.synchronize()
    _attention(rng, plan.q_re, plan.k_re, plan.v_re, plan.kv_valid, o, lse, do_re, delta, dq, dk, dv, plan.qstart,
               plan.qlen, plan.qcols, plan.klists, BH, Nt, D, sm)
    del plan, o, lse, dq, dk, dv, do_re, gd, inp
    torch.cuda.empty_cache()


def test_full_size_cross_v2a():
    """The v2a bridge cross-attention at config-4 size (hymm/config.py:249-253:
    Q = audio, 1-D chunks of 64 tokens; K = video, 3-D 4x4x4 chunks; sparsity
    0.875): 2,000 audio queries over the 302,400 video keys of config 4."""
    import bench
    from prism_amd import ops
    from prism_amd.uniform_block_attention import plan_chunked

    say("fullsize v2a: inputs")
    inp = bench.make_inputs("c4")
    B, H, D, grid = inp["B"], inp["H"], inp["D"], inp["grid"]
    BH, sm, Sa, sp = B * H, 1 / math.sqrt(D), 2000, 0.875
    gen = torch.Generator(device=DEV).manual_seed(7)
    qa = torch.randn((B, H, Sa, D), generator=gen, device=DEV).to(torch.bfloat16)
    do = torch.randn((B, H, Sa, D), generator=gen, device=DEV).to(torch.bfloat16)
    lq = ops.ChunkLayout((1, 1, Sa), (1, 1, 64), DEV)
    lk = ops.ChunkLayout(grid, (4, 4, 4), DEV)
    say("fullsize v2a: plan")
    plan = plan_chunked(qa, inp["k"], inp["v"], lq, lk, sparsity=sp, cdf_threshold=None, sm_scale=sm,
                        keep_scores=True)
    Ntq, Ntk = lq.Nt, lk.Nt
    k_tile_count = plan.kv_valid.view(-1, TILE).sum(1, dtype=torch.int32)
    q_tile_count = torch.clamp(Sa - TILE * torch.arange(Ntq, device=DEV), 0, TILE).to(torch.int32)
    tiles, ntiles, tcap = plan.sel["tiles"], plan.sel["ntiles"], plan.sel["tcap"]
    rng = np.random.default_rng(6)
    kbt = O.chunk_kblock_tiles(lk.N_b, lk.csz, Ntk)
    _selection_rows(rng, plan.scores.view(BH, lq.N_b, lk.N_b), tiles, ntiles, tcap, sp, None, sm, kbt, Ntk,
                    k_tile_count.cpu().numpy())
    _list_structure(tiles, ntiles, tcap, Ntk, lq.N_b, BH, lq.block_id_of_tile, plan.qstart, plan.qlen,
                    q_tile_count)

    say("fullsize v2a: forward")
    o, lse = ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qunion, sm, plan.qpair, plan.qorder)
    say("fullsize v2a: backward")
    gd = ops.chunk_gather_pool(do, lq, None, rows=True, dot_with=o)
    do_re, delta = gd["rows"], gd["rowdot"]
    kunion = plan.key_lists()
    m2 = ops.lse_to_m2(lse)
    dq, dk, dv = ops.bsa_bwd(plan.q_re, plan.k_re, plan.v_re, do_re, m2, delta, plan.kv_valid, plan.tmasks,
                             plan.qunion, kunion, sm, plan.qpair, plan.kpair, plan.qorder, plan.korder)
    torch.cuda.synchronize()
    _attention(rng, plan.q_re, plan.k_re, plan.v_re, plan.kv_valid, o, lse, do_re, delta, dq, dk, dv, plan.qstart,
               plan.qlen, plan.qcols, plan.klists, BH, Ntq, D, sm)
    del plan, o, lse, dq, dk, dv, do_re, gd, inp
    torch.cuda.empty_cache()
