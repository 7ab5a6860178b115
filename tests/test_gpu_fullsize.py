"""Parity at the full sizes of the BASELINE GPU configs:
  c4  2K:    B=1, H=5,  D=128, input grid 21x90x160, top-48 + p = 0.9
  c3  1080p: B=1, H=24, D=128, input grid 21x68x120, top-32 + p = 0.9
  c2  720p:  B=1, H=24, D=128, input grid 21x45x80,  sparsity 0.75
(inputs from bench.make_inputs, the benchmark's own generator).

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
    each query row's LSE and delta taken from the kernels (the LSE itself is
    checked on the sampled query rows);
  * two forward launches give bit-identical O and LSE.
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


def _tol(got, ref, what):
    """max-abs 2e-2, mean-abs 2e-3 (bf16 vs float64)."""
    err = np.abs(got.astype(np.float64) - ref)
    mx, mean = float(err.max()), float(err.mean())
    say(what, "max-abs", mx, "mean-abs", mean)
    assert mx <= 2e-2 and mean <= 2e-3, (what, mx, mean)


def _rows(t, bh, first, count):
    """Rows [first, first + count) of head bh of a [B, H, S, D] tile-order tensor, as float32 numpy."""
    return t.view(-1, t.shape[-2], t.shape[-1])[bh, first:first + count].float().cpu().numpy()


@pytest.mark.parametrize("cfg", ["c2", "c3", "c4"])
def test_full_size(cfg):
    import bench
    from prism_amd import a2v_token_norms, ops, plan_dynamic
    from prism_amd.adapter import padded_grid
    from prism_amd.dynamic_block_shape import _gradient_and_shapes

    say("fullsize:", cfg, "inputs")
    inp = bench.make_inputs(cfg)
    B, H, D, grid = inp["B"], inp["H"], inp["D"], inp["grid"]
    gp, _ = padded_grid(grid)
    BH, sm = B * H, 1 / math.sqrt(D)
    say("fullsize: plan")
    norms = a2v_token_norms(inp["res"])
    with torch.no_grad():
        sid = _gradient_and_shapes(inp["v"], norms, gp, "ivpq", 0.5, 0.15, 1.0, None, grid)[2]
        N_b = ops.ZoneLayout(sid, gp, grid).N_b
        if inp["sp_only"] is not None:
            sp, cdf = inp["sp_only"], None
        else:
            sp, cdf = 1.0 - (inp["topk"] + 0.5) / N_b, inp["cdf"]
        plan = plan_dynamic(inp["q"], inp["k"], inp["v"], gp, method="ivpq", sparsity=sp, cdf_threshold=cdf,
                            audio_token_norms=norms, input_grid=grid)
    lay, Nt = plan.lay, plan.lay.Nt
    assert lay.N_b == N_b and plan.S == gp[0] * gp[1] * gp[2]
    tiles, ntiles, tcap = plan.sel["tiles"], plan.sel["ntiles"], plan.sel["tcap"]

    # ---- selection of sampled score rows vs the oracle (bit-exact)
    say("fullsize: selection of sampled rows")
    rng = np.random.default_rng(4)
    rows = np.sort(rng.choice(BH * N_b, 48, replace=False))
    ridx = torch.as_tensor(rows, device=DEV)
    sc = plan.scores.reshape(BH * N_b, N_b)[ridx].cpu().numpy()
    sel, nsel = O.select(sc, sp, cdf, sm)
    _, kbt, nb, _ = O.tile_maps(lay.shape_ids.cpu().numpy())
    assert nb == N_b
    tc = plan.tile_count.cpu().numpy()
    ref_tiles, ref_n = O.expand_tiles(sel, nsel, kbt, Nt, tc)
    got_n = ntiles.view(-1)[ridx].cpu().numpy()
    got_t = tiles.view(BH * N_b, tcap)[ridx].cpu().numpy()
    assert np.array_equal(got_n, ref_n)
    for i in range(len(rows)):
        assert np.array_equal(got_t[i, : got_n[i]], ref_tiles[i, : ref_n[i]]), rows[i]

    # ---- every list: strictly ascending in [0, Nt); query tile -> block row
    say("fullsize: list structure")
    t2 = tiles.view(BH * N_b, tcap)
    live = torch.arange(tcap, device=DEV)[None, :] < ntiles.view(-1, 1)
    assert bool(((t2 >= 0) & (t2 < Nt) | ~live).all())
    assert bool(((t2[:, 1:] > t2[:, :-1]) | ~live[:, 1:]).all())
    del live
    brow = (torch.arange(BH, device=DEV)[:, None] * N_b + lay.block_id_of_tile.long()[None, :]).reshape(-1)
    assert torch.equal(plan.qstart, brow * tcap)
    want_len = torch.where(plan.tile_count.repeat(BH) == 0, 0, ntiles.view(-1)[brow])
    assert torch.equal(plan.qlen.long(), want_len.long())
    say("fullsize: kept tile pairs", int(plan.qlen.sum()))

    # ---- forward (twice) and backward at full size
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
    torch.cuda.synchronize()
    kv = plan.kv_valid.cpu().numpy().astype(bool)
    lse_h = lse.view(BH, -1)
    delta_h = delta.view(BH, -1)

    # ---- sampled query tiles: O, LSE, dQ vs the float64 oracle
    qlen = plan.qlen.cpu().numpy()
    qstart = plan.qstart.cpu().numpy()
    cand = np.nonzero(qlen > 0)[0]
    pick = list(rng.choice(cand, 5, replace=False)) + [int(cand[np.argmax(qlen[cand])])]
    for r in pick:
        bh, t = divmod(int(r), Nt)
        n = int(qlen[r])
        say("fullsize: query tile", bh, t, "keys", n)
        cols = plan.qcols[int(qstart[r]): int(qstart[r]) + n].cpu().numpy()
        keys = O._row_keys(cols, 0, n)
        kidx = torch.as_tensor(keys, device=DEV)
        # tile 0 of the oracle's sequence holds the queries, tiles 1..n the listed keys
        Sx = TILE * (n + 1)
        qx, kx, vx, dox = (np.zeros((1, Sx, D), np.float32) for _ in range(4))
        qx[0, :TILE] = _rows(plan.q_re, bh, t * TILE, TILE)
        dox[0, :TILE] = _rows(do_re, bh, t * TILE, TILE)
        kx[0, TILE:] = plan.k_re.view(BH, -1, D)[bh][kidx].float().cpu().numpy()
        vx[0, TILE:] = plan.v_re.view(BH, -1, D)[bh][kidx].float().cpu().numpy()
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

    # ---- sampled key tiles: dK, dV summed over all query tiles that list them
    kstart, klen, kcols = (x.cpu().numpy() for x in klists)
    kcand = np.nonzero(klen > 0)[0]
    kpick = list(rng.choice(kcand, 2, replace=False)) + [int(kcand[np.argmax(klen[kcand])])]
    for r in kpick:
        bh, j = divmod(int(r), Nt)
        n = int(klen[r])
        say("fullsize: key tile", bh, j, "query tiles", n)
        qt = kcols[int(kstart[r]): int(kstart[r]) + n].astype(np.int64)
        qrows = (qt[:, None] * TILE + np.arange(TILE)[None, :]).reshape(-1)
        qi = torch.as_tensor(qrows, device=DEV)
        Qs = plan.q_re.view(BH, -1, D)[bh][qi].double().cpu().numpy()
        dOs = do_re.view(BH, -1, D)[bh][qi].double().cpu().numpy()
        Ls = lse_h[bh][qi].double().cpu().numpy()
        dls = delta_h[bh][qi].double().cpu().numpy()
        Kj = _rows(plan.k_re, bh, j * TILE, TILE).astype(np.float64)
        Vj = _rows(plan.v_re, bh, j * TILE, TILE).astype(np.float64)
        s = Qs @ Kj.T * sm
        s[:, ~kv[j * TILE:(j + 1) * TILE]] = -np.inf
        p = np.zeros_like(s)
        ok = np.isfinite(Ls)
        p[ok] = np.exp(s[ok] - Ls[ok, None])
        ds = p * (dOs @ Vj.T - dls[:, None])
        _tol(_rows(dk, bh, j * TILE, TILE), ds.T @ Qs * sm, "dK")
        _tol(_rows(dv, bh, j * TILE, TILE), p.T @ dOs, "dV")
    del plan, o, lse, dq, dk, dv, do_re, gd, inp
    torch.cuda.empty_cache()
