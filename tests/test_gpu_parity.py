"""GPU parity: every HIP stage against the CPU oracle on identical seeded inputs.

Bit-exact: zone statistics, gradients, shape ids, audio statistics, A2V norms,
geometry, pooled block means, fp32 scores, selected sets / tile lists, list
transpose.  Tolerance (bf16 vs float64 oracle): attention O, dQ, dK, dV with
max-abs 2e-2 and mean-abs 2e-3.
"""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.cases import bf16, padded_case

pytestmark = pytest.mark.gpu

DEV = "cuda"


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def dev(x: np.ndarray) -> torch.Tensor:
    if x.dtype == np.uint16:
        return torch.from_numpy(x.view(np.int16).copy()).view(torch.bfloat16).to(DEV)
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def host(t: torch.Tensor) -> np.ndarray:
    t = t.detach()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    if a.dtype == np.float32:
        return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.astype(np.float32).view(np.uint32))
    return a.shape == b.shape and np.array_equal(a, b)


CASES = [
    # (name, seed, B, H, grid_real, D, dtype, lowrank, audio)
    ("c1_fp32_d64", 0, 1, 4, (4, 16, 16), 64, "f32", False, 64),
    ("bf16_d128_lowrank", 1, 1, 3, (13, 20, 24), 128, "bf16", True, 32),
    ("bf16_d128_nopad", 2, 2, 2, (8, 16, 16), 128, "bf16", False, 0),
]


def make(case):
    name, seed, B, H, gr, D, dt, lowrank, audio = case
    c = padded_case(seed, B, H, gr, D, lowrank=lowrank, audio_tokens=audio)
    conv = bf16 if dt == "bf16" else (lambda x: x)
    c["qh"], c["kh"], c["vh"] = conv(c["q"]), conv(c["k"]), conv(c["v"])
    c["nh"] = None if c["norms"] is None else conv(c["norms"])
    c["pad"] = tuple(gr) != tuple(c["grid"])
    c["lowrank"] = lowrank
    return c


@pytest.fixture(scope="module", params=CASES, ids=[c[0] for c in CASES])
def case(request):
    say(request.param)
    return make(request.param)


def test_zone_stats_bitexact(case):
    from prism_amd import ops
    valid = case["valid"] if case["pad"] else None
    p_ref, av_ref = O.zone_stats(case["vh"], case["grid"], valid)
    p, av = ops.zone_stats(dev(case["vh"]), case["grid"], None if valid is None else dev(valid))
    assert bits_equal(host(p), p_ref)
    assert np.array_equal(host(av), av_ref)


def test_zone_gradient_shapes_bitexact(case):
    from prism_amd import ops
    valid = case["valid"] if case["pad"] else None
    D = case["q"].shape[-1]
    p_ref, av_ref = O.zone_stats(case["vh"], case["grid"], valid)
    rho_ref, an_ref = O.zone_gradient(p_ref, av_ref, D)
    rho, an = ops.zone_gradient(dev(p_ref), dev(av_ref), D)
    assert bits_equal(host(rho), rho_ref)
    assert bits_equal(host(an), an_ref)
    ab = vh = ab_d = vh_d = None
    if case["nh"] is not None:
        ab, vh = O.audio_zone_stats(case["nh"], case["grid"], valid)
        ab_d, vh_d = ops.audio_zone_stats(dev(case["nh"]), case["grid"], None if valid is None else dev(valid))
        assert bits_equal(host(ab_d), ab)
        assert bits_equal(host(vh_d), vh)
    for method in ("ivpq", "penalty"):
        for tau in (0.15, 0.6, 1.5):
            g_ref, r_ref, s_ref = O.zone_shapes(rho_ref, an_ref, ab, vh, method, 0.5, tau, 1.0)
            g, r, s = ops.zone_shapes(dev(rho_ref), dev(an_ref), None if ab is None else dev(ab),
                                      None if vh is None else dev(vh), method, 0.5, tau, 1.0)
            assert bits_equal(host(g), g_ref)
            assert bits_equal(host(r), r_ref)
            assert np.array_equal(host(s), s_ref), (method, tau)


def test_a2v_norms_bitexact():
    from prism_amd import ops
    rng = np.random.default_rng(5)
    for S, C, dt in ((300, 256, "f32"), (257, 5120, "bf16"), (64, 3072, "bf16"), (10, 8, "f32")):
        say("a2v", S, C, dt)
        x = rng.standard_normal((1, S, C)).astype(np.float32)
        xh = bf16(x) if dt == "bf16" else x
        ref = O.a2v_norms(xh[0], dt == "bf16")
        got = host(ops.a2v_norms(dev(xh)))
        vt = np.uint32 if dt == "f32" else np.uint16
        assert np.array_equal(got.view(vt), ref.view(vt))


def _shape_ids_for(case, method="ivpq"):
    valid = case["valid"] if case["pad"] else None
    return O.select_zone_shapes(case["vh"], case["nh"], case["grid"], method, 0.5, 0.15, 1.0, valid)


def test_layout_and_rearrange(case):
    from prism_amd import ops
    sid = _shape_ids_for(case)
    # exercise every candidate shape as well
    sid_all = np.arange(len(sid)) % 13
    for s in (sid, sid_all):
        src_ref, inv_ref = O.rearrange_index(s, case["grid"])
        src, inv = ops.rearrange_index(dev(s), case["grid"])
        assert np.array_equal(host(src), src_ref) and np.array_equal(host(inv), inv_ref)
        bot, kbt, nb, boff = O.tile_maps(s)
        lay = ops.ZoneLayout(dev(s), case["grid"])
        assert lay.N_b == nb
        assert np.array_equal(host(lay.block_id_of_tile), bot)
        assert np.array_equal(host(lay.block_offset)[:-1], boff)
        first = host(lay.block_first_tile)[: nb + 1]
        assert np.array_equal(first[:-1], kbt[:nb, 0]) and first[-1] == len(bot)


def test_gather_pool_bitexact(case):
    from prism_amd import ops
    sid = np.arange(case["grid"][0] // 8 * case["grid"][1] // 8 * case["grid"][2] // 8) % 13
    valid = case["valid"] if case["pad"] else None
    lay = ops.ZoneLayout(dev(sid), case["grid"])
    vd = None if valid is None else dev(valid)
    for name in ("qh", "kh"):
        x = case[name]
        ref, bc, tc = O.block_pool(x, sid, case["grid"], valid)
        g = ops.gather_pool(dev(x), lay, vd, rows=True, pool=True, counts=True)
        assert bits_equal(host(g["block_mean"]), ref)
        assert np.array_equal(host(g["block_count"]), bc)
        assert np.array_equal(host(g["tile_count"]), tc)
        src, _ = O.rearrange_index(sid, case["grid"])
        xf = x if x.dtype == np.uint16 else bf16(x)
        assert np.array_equal(host(g["rows"]), xf[:, :, src])
        vre = np.ones(len(src), np.uint8) if valid is None else valid[src]
        assert np.array_equal(host(g["valid_re"]), vre)


def test_scores_bitexact():
    from prism_amd import ops
    rng = np.random.default_rng(7)
    for BH, N, D in ((2, 200, 64), (1, 333, 128), (3, 128, 128)):
        say("scores", BH, N, D)
        qc = rng.standard_normal((BH, N, D)).astype(np.float32)
        kc = rng.standard_normal((BH, N, D)).astype(np.float32)
        bc = (rng.random(N) > 0.1).astype(np.int32)
        ref = O.block_scores(qc, kc, bc)
        got = host(ops.block_scores(dev(qc), dev(kc), dev(bc)))
        assert bits_equal(got, ref)


def _random_scores(rng, rows, N, kind):
    s = rng.standard_normal((rows, N)).astype(np.float32) * 3
    if kind == "ties":
        s = np.round(s * 2) / 2
    if kind == "neginf":
        s[:, rng.random(N) < 0.2] = -np.inf
    if kind == "peaked":
        s[:, : N // 10] += 8
    return s


@pytest.mark.parametrize("kind", ["plain", "ties", "neginf", "peaked"])
def test_select_bitexact(kind):
    from prism_amd import ops
    rng = np.random.default_rng(11)
    # one wave per row (16 to 96 elements per lane, full and partial last
    # slots), then one workgroup per row (6,145 to 16,384 blocks)
    for N in (37, 300, 1024, 1440, 2900, 4097, 5328, 6144, 6145, 6500):
        rows = 24
        s = _random_scores(rng, rows, N, kind)
        first = np.arange(N + 1, dtype=np.int32)
        for sp, p in ((0.9, None), (None, 0.9), (1 - 5.5 / N, 0.9), (0.5, 0.3), (None, 0.2)):
            say("select", kind, N, sp, p)
            ref_sel, ref_n = O.select(s, sp, p, 0.125)
            res = ops.select_tiles(dev(s), sp, p, 0.125, dev(first), None, want_blocks=True)
            n = host(res["nsel"])
            assert np.array_equal(n, ref_n), (kind, N, sp, p)
            got = host(res["sel_blocks"])
            for r in range(rows):
                assert np.array_equal(got[r, : n[r]], ref_sel[r, : n[r]]), (kind, N, sp, p, r)


@pytest.mark.parametrize("N", [300, 5000, 6144, 6500])
def test_select_tile_expansion_any_tile_count(N):
    """Blocks of 0..4 tiles (the C-ABI takes any block_first_tile) with padded
    tiles dropped: each row's list is the tiles of its selected blocks, in
    ascending block order, whose tile_count is non-zero."""
    from prism_amd import ops
    rng = np.random.default_rng(5)
    rows = 16
    s = _random_scores(rng, rows, N, "plain")
    per = rng.integers(0, 5, N)
    first = np.concatenate([[0], np.cumsum(per)]).astype(np.int32)
    tc = (rng.random(int(first[-1])) > 0.2).astype(np.int32)
    for sp, p in ((0.9, None), (None, 0.9), (0.5, 0.3)):
        say("expansion", N, sp, p)
        ref_sel, ref_n = O.select(s, sp, p, 0.125)
        res = ops.select_tiles(dev(s), sp, p, 0.125, dev(first), dev(tc), want_blocks=True, tiles_per_block=4)
        nt, tiles = host(res["ntiles"]), host(res["tiles"])
        assert np.array_equal(host(res["nsel"]), ref_n)
        for r in range(rows):
            want = [t for b in ref_sel[r, : ref_n[r]] for t in range(first[b], first[b + 1]) if tc[t] > 0]
            assert nt[r] == len(want), (N, sp, p, r)
            assert np.array_equal(tiles[r, : nt[r]], want), (N, sp, p, r)


def test_select_row_of_65536_tiles():
    """The widest register-held rows (16,384 blocks) with 4 tiles per block
    and every block selected: 65,536 tiles in one row, more than a 16-bit
    count holds.  Tiles, blocks and both counts are exact."""
    from prism_amd import ops
    rng = np.random.default_rng(17)
    N, rows = 16384, 3
    s = _random_scores(rng, rows, N, "plain")
    first = (4 * np.arange(N + 1)).astype(np.int32)
    for sp, p in ((0.0, None), (0.0, 0.999999)):
        say("select 65536 tiles", sp, p)
        ref_sel, ref_n = O.select(s, sp, p, 0.125)
        assert (ref_n == N).all()
        res = ops.select_tiles(dev(s), sp, p, 0.125, dev(first), None, want_blocks=True, tiles_per_block=4)
        assert res["tcap"] == 4 * N
        n, nt = host(res["nsel"]), host(res["ntiles"])
        assert (n == N).all() and (nt == 4 * N).all(), (n, nt)
        got, tiles = host(res["sel_blocks"]), host(res["tiles"])
        for r in range(rows):
            assert np.array_equal(got[r], np.arange(N))
            assert np.array_equal(tiles[r], np.arange(4 * N))


@pytest.mark.parametrize("kind", ["plain", "ties", "neginf", "peaked"])
def test_select_bitexact_wide_rows(kind):
    """Rows of more than 16384 blocks (the pass-by-pass workgroup kernel):
    bit-exact against the oracle in all three modes, with blocks of 0-3 tiles
    and padded tiles dropped."""
    from prism_amd import ops
    rng = np.random.default_rng(13)
    for N in (16385, 23000, 70000):
        rows = 6
        s = _random_scores(rng, rows, N, kind)
        per = rng.integers(0, 4, N)
        first = np.concatenate([[0], np.cumsum(per)]).astype(np.int32)
        tc = (rng.random(int(first[-1])) > 0.2).astype(np.int32)
        for sp, p in ((0.9, None), (None, 0.9), (1 - 5.5 / N, 0.9), (0.5, 0.3), (None, 0.2)):
            say("select wide", kind, N, sp, p)
            ref_sel, ref_n = O.select(s, sp, p, 0.125)
            res = ops.select_tiles(dev(s), sp, p, 0.125, dev(first), dev(tc), want_blocks=True, tiles_per_block=3)
            n, got = host(res["nsel"]), host(res["sel_blocks"])
            assert np.array_equal(n, ref_n), (kind, N, sp, p)
            nt, tiles = host(res["ntiles"]), host(res["tiles"])
            for r in range(rows):
                assert np.array_equal(got[r, : n[r]], ref_sel[r, : n[r]]), (kind, N, sp, p, r)
                want = np.concatenate([np.arange(first[b], first[b + 1]) for b in ref_sel[r, : n[r]]] + [np.zeros(0, int)])
                want = want[tc[want] > 0] if want.size else want
                assert nt[r] == want.size, (kind, N, sp, p, r)
                assert np.array_equal(tiles[r, : nt[r]], want), (kind, N, sp, p, r)


def test_select_tile_expansion_bitexact(case):
    from prism_amd import ops
    sid = _shape_ids_for(case)
    valid = case["valid"] if case["pad"] else None
    r = O.select_pipeline(case["qh"], case["kh"], case["vh"], case["grid"], sparsity=0.75, cdf_threshold_p=0.9,
                          audio_norms=case["nh"], valid=valid, shape_ids=sid)
    lay = ops.ZoneLayout(dev(sid), case["grid"])
    res = ops.select_tiles(dev(r["scores"]), 0.75, 0.9, 1 / math.sqrt(case["q"].shape[-1]), lay.block_first_tile,
                           None if valid is None else dev(r["tile_count"]))
    nt = host(res["ntiles"])
    assert np.array_equal(nt, r["ntiles"])
    tiles = host(res["tiles"])
    for i in range(len(nt)):
        assert np.array_equal(tiles[i, : nt[i]], r["tiles"][i, : nt[i]])


def test_full_selection_pipeline_bitexact(case):
    """plan_dynamic (stats -> shapes -> pooling -> scores -> selection) vs the
    oracle pipeline on the same inputs."""
    from prism_amd import plan_dynamic
    valid = case["valid"] if case["pad"] else None
    D = case["q"].shape[-1]
    for method, sp, p in (("ivpq", 0.75, 0.9), ("penalty", 0.5, None), ("ivpq", None, 0.5)):
        say("pipeline", method, sp, p)
        ref = O.select_pipeline(case["qh"], case["kh"], case["vh"], case["grid"], method=method, sparsity=sp,
                                cdf_threshold_p=p, audio_norms=case["nh"], valid=valid, skip_padded_queries=True)
        plan = plan_dynamic(dev(case["qh"]), dev(case["kh"]), dev(case["vh"]), case["grid"], method=method,
                            sparsity=sp, cdf_threshold=p,
                            audio_token_norms=None if case["nh"] is None else dev(case["nh"]),
                            valid_mask=None if valid is None else dev(valid).bool(), keep_scores=True)
        assert np.array_equal(host(plan.lay.shape_ids), ref["shape_ids"])
        assert bits_equal(host(plan.scores).reshape(ref["scores"].shape), ref["scores"])
        qlen = host(plan.qlen)
        assert np.array_equal(qlen, ref["qlen"])
        qs, qc = host(plan.qstart), host(plan.qcols)
        for i in range(len(qlen)):
            assert np.array_equal(qc[qs[i]: qs[i] + qlen[i]], ref["qcols"][ref["qstart"][i]: ref["qstart"][i] + qlen[i]])
        assert D in (64, 128)


def test_transpose_lists_bitexact(case):
    from prism_amd import ops, plan_dynamic
    valid = case["valid"] if case["pad"] else None
    plan = plan_dynamic(dev(case["qh"]), dev(case["kh"]), dev(case["vh"]), case["grid"], method="ivpq",
                        sparsity=0.7, cdf_threshold=0.9, valid_mask=None if valid is None else dev(valid).bool())
    BH = plan.B * plan.H
    Nt = plan.lay.Nt
    ks, kl, kc = ops.transpose_lists(plan.qstart, plan.qlen, plan.qcols, BH, Nt)
    ref_c, ref_l = O.transpose_lists(host(plan.qstart), host(plan.qlen), host(plan.qcols), BH, Nt)
    kl = host(kl)
    assert np.array_equal(kl, ref_l)
    kc = host(kc).reshape(BH * Nt, Nt)
    for i in range(BH * Nt):
        assert np.array_equal(kc[i, : kl[i]], ref_c[i, : kl[i]])


def test_pair_union_bitexact(case):
    """prism_pair_union on the plan's query-tile lists (with key-validity
    words) and on the transposed key-tile lists vs the oracle's set union."""
    from prism_amd import ops, plan_dynamic
    valid = case["valid"] if case["pad"] else None
    B, H, S, D = case["q"].shape
    plan = plan_dynamic(dev(case["qh"]), dev(case["kh"]), dev(case["vh"]), case["grid"], method="ivpq",
                        sparsity=0.6, cdf_threshold=0.9, valid_mask=None if valid is None else dev(valid).bool())
    Nt = plan.lay.Nt
    tm = None if plan.tmasks is None else host(plan.tmasks).view(np.uint64)
    if valid is not None:
        assert np.array_equal(tm, O.tile_masks(host(plan.kv_valid)))
    klists = ops.transpose_lists(plan.qstart, plan.qlen, plan.qcols, B * H, Nt)
    for lists, masks in (((plan.qstart, plan.qlen, plan.qcols), tm), (klists, None)):
        st, ln, cl = (host(t) for t in lists)
        # the pairing of each group of 8 tiles, and the unions with and without it
        pm = ops.pair_tiles(*lists, Nt)
        pm_ref = O.pair_tiles(st, ln, cl, Nt)
        assert np.array_equal(host(pm), pm_ref)
        for pairmap, pref in ((None, None), (pm, pm_ref)):
            ustart, ulen, ucols = ops.pair_union(*lists, Nt, None if masks is None else plan.tmasks, pairmap=pairmap)
            ref = O.pair_union(st, ln, cl, Nt, masks, pref)
            ulen, ustart, ucols = host(ulen), host(ustart), host(ucols)
            assert len(ref) == len(ulen)
            for p, r in enumerate(ref):
                assert ulen[p] == len(r)
                assert np.array_equal(ucols[ustart[p]: ustart[p] + ulen[p]], r)
        # the pairing never lengthens the work lists
        assert int(host(ops.pair_union(*lists, Nt, pairmap=pm)[1]).sum()) <= int(host(ops.pair_union(*lists, Nt)[1]).sum())


def test_lse_to_m2():
    from prism_amd import ops
    x = torch.tensor([0.0, -1.5, 3.25, -float("inf"), 80.0], device=DEV)
    m2 = host(ops.lse_to_m2(x))
    ref = np.array([0.0, -1.5, 3.25, np.inf, 80.0], np.float32) * np.float32(1.4426950408889634)
    ref[3] = np.inf
    assert np.array_equal(m2, ref.astype(np.float32))


def _xcd_group_remap(bid, n, G):
    """The attention kernels' default workgroup mapping, restated."""
    full = n // (8 * G) * (8 * G)
    if bid >= full:
        return bid
    chunk, xcd, slot = bid // (8 * G), bid & 7, (bid >> 3) % G
    return chunk * 8 * G + xcd * G + slot


def _check_order(order, ulen, G, tail):
    """prism_pair_order: a permutation; ids before the tail keep the default
    mapping; the tail holds the same pairs, longest list first (ties: lower pair)."""
    n = len(ulen)
    assert np.array_equal(np.sort(order), np.arange(n))
    k = n - tail
    base = np.array([_xcd_group_remap(b, n, G) for b in range(n)])
    assert np.array_equal(order[:k], base[:k])
    want = sorted(base[k:].tolist(), key=lambda p: (-int(ulen[p]), p))
    assert order[k:].tolist() == want


def _bf16_half_ulp(x):
    """Half a bf16 ulp at |x| (8 significant bits: 2^(e - 8) for |x| in
    [2^e, 2^(e + 1))); 0 at 0."""
    a = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    return np.where(a > 0, np.exp2(e - 8), 0.0)


def _tol(got, ref, what, rel_bound=1e-2, slack=None):
    """max-abs 2e-2, mean-abs 2e-3 (bf16 vs float64); plus
    a relative bound ||got - ref|| / ||ref|| <= 1e-2 (Frobenius), which
    catches a scaled result where the values are small (at long lists |O| and
    |dQ| average ~6e-3, below the absolute bounds).

    Both absolute bounds apply to the error beyond a per-element allowance
    for bf16: half a bf16 ulp of ref[i] (a result stored in bf16 differs from
    the exact value by up to that much even when computed exactly) plus
    `slack`.  So max(|err_i| - allow_i) <= 2e-2 and mean(|err_i| - allow_i)
    <= 2e-3.  At |value| >= 8 the half ulp (0.031) alone exceeds 2e-2
    (gradients of queries that keep one key tile reach |dK| ~ 12), and where
    gradients average ~1 (cross attention with few queries per key) the
    reference's own bf16 arithmetic has a mean-abs error of 2.5e-3.  Below
    |value| = 1 the half ulp is at most 2^-9, so at the north-star inputs'
    scale the bounds are the plain ones.

    slack: a further per-element allowance (the rounding bound of bf16
    operands in sums whose terms cancel, from the oracle's term magnitudes)."""
    diff = got.astype(np.float64) - ref
    err = np.abs(diff)
    mx, mean = float(err.max()), float(err.mean())
    allow = _bf16_half_ulp(ref) + (0.0 if slack is None else slack)
    excess = float((err - allow).max())
    mean_excess = float((err - allow).mean())
    ref_norm = float(np.linalg.norm(ref))
    rel = float(np.linalg.norm(diff)) / ref_norm if ref_norm > 0 else float(np.linalg.norm(diff))
    say(what, "max-abs", mx, "beyond bf16 allowance", excess, "mean-abs", mean, "beyond allowance", mean_excess,
        "rel", rel, "||ref||", ref_norm, "max|ref|", float(np.abs(ref).max()))
    assert excess <= 2e-2 and mean_excess <= 2e-3, (what, mx, excess, mean, mean_excess)
    assert rel <= rel_bound, (what, "relative error", rel, "||ref||", ref_norm)


def test_attention_fwd_bwd_tolerance(case):
    """O, LSE, dQ, dK, dV of the MFMA kernels vs the float64 oracle on the
    same bf16 tile-order inputs and the same lists."""
    from prism_amd import ops, plan_dynamic
    valid = case["valid"] if case["pad"] else None
    B, H, S, D = case["q"].shape
    sm = 1 / math.sqrt(D)
    plan = plan_dynamic(dev(case["qh"]), dev(case["kh"]), dev(case["vh"]), case["grid"], method="ivpq",
                        sparsity=0.6, cdf_threshold=0.9, valid_mask=None if valid is None else dev(valid).bool())
    o, lse = ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qunion, sm, plan.qpair)
    # the tile pairing changes no bit: neighbouring pairs give the same O and LSE
    q0 = ops.pair_union(plan.qstart, plan.qlen, plan.qcols, plan.lay.Nt, plan.tmasks)
    o0, lse0 = ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, q0, sm)
    assert bits_equal(host(o), host(o0)) and bits_equal(host(lse), host(lse0))
    # nor does the launch order (every tail length, up to all workgroups)
    npairs = plan.qunion[1].numel()
    for frac in (0.1, 1.0):
        qo = ops.pair_order(plan.qunion[1], 64, frac)
        _check_order(host(qo), host(plan.qunion[1]), 64, min(npairs, 16384, int(npairs * frac)))
        o1, lse1 = ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qunion, sm, plan.qpair, qo)
        assert bits_equal(host(o), host(o1)) and bits_equal(host(lse), host(lse1))
    qf = O.bf16_bits_to_f32(host(plan.q_re)).reshape(B * H, S, D)
    kf = O.bf16_bits_to_f32(host(plan.k_re)).reshape(B * H, S, D)
    vf = O.bf16_bits_to_f32(host(plan.v_re)).reshape(B * H, S, D)
    kv = None if plan.kv_valid is None else host(plan.kv_valid)
    lists = (host(plan.qstart), host(plan.qlen), host(plan.qcols))
    o_ref, lse_ref = O.attn_fwd(qf, kf, vf, *lists, kv, sm)
    og = O.bf16_bits_to_f32(host(o)).reshape(B * H, S, D)
    _tol(og, o_ref, "O")
    lg = host(lse).reshape(B * H, S)
    fin = np.isfinite(lse_ref)
    assert np.array_equal(np.isfinite(lg), fin)
    assert np.abs(lg[fin] - lse_ref[fin]).max() < 1e-3
    # backward with a seeded dO
    rng = np.random.default_rng(99)
    do = bf16(rng.standard_normal((B, H, S, D)).astype(np.float32))
    do_t = dev(do)
    delta = ops.bwd_preprocess(o, do_t)
    klists = ops.transpose_lists(plan.qstart, plan.qlen, plan.qcols, B * H, plan.lay.Nt)
    kpair = ops.pair_tiles(*klists, plan.lay.Nt)
    kunion = ops.pair_union(*klists, plan.lay.Nt, pairmap=kpair)
    m2 = ops.lse_to_m2(lse)
    dq, dk, dv = ops.bsa_bwd(plan.q_re, plan.k_re, plan.v_re, do_t, m2, delta, plan.kv_valid,
                             plan.tmasks, plan.qunion, kunion, sm, plan.qpair, kpair)
    grads0 = ops.bsa_bwd(plan.q_re, plan.k_re, plan.v_re, do_t, m2, delta, plan.kv_valid, plan.tmasks, q0,
                         ops.pair_union(*klists, plan.lay.Nt), sm)
    for g, g0 in zip((dq, dk, dv), grads0):
        assert bits_equal(host(g), host(g0))
    korder = ops.pair_order(kunion[1], 32, 1.0)
    _check_order(host(korder), host(kunion[1]), 32, min(kunion[1].numel(), 16384))
    grads1 = ops.bsa_bwd(plan.q_re, plan.k_re, plan.v_re, do_t, m2, delta, plan.kv_valid, plan.tmasks, plan.qunion,
                         kunion, sm, plan.qpair, kpair, ops.pair_order(plan.qunion[1], 64, 1.0), korder)
    for g, g1 in zip((dq, dk, dv), grads1):
        assert bits_equal(host(g), host(g1))
    dof = O.bf16_bits_to_f32(do).reshape(B * H, S, D)
    dq_r, dk_r, dv_r = O.attn_bwd(qf, kf, vf, og, dof, lse_ref, *lists, kv, sm)
    for name, g, r in (("dQ", dq, dq_r), ("dK", dk, dk_r), ("dV", dv, dv_r)):
        _tol(O.bf16_bits_to_f32(host(g)).reshape(B * H, S, D), r, name)


def test_debug_mode_checks_lists(case, monkeypatch):
    """PRISM_DEBUG=1: the attention entry points copy their work lists to the
    host and check them before launching.  Valid lists give the same bits as
    without the checks; corrupted ones (kept inside the operands' bounds,
    so a launch could not fault) raise ValueError naming the defect."""
    from prism_amd import ops, plan_dynamic
    valid = case["valid"] if case["pad"] else None
    B, H, S, D = case["q"].shape
    sm = 1 / math.sqrt(D)
    plan = plan_dynamic(dev(case["qh"]), dev(case["kh"]), dev(case["vh"]), case["grid"], method="ivpq",
                        sparsity=0.6, cdf_threshold=0.9, valid_mask=None if valid is None else dev(valid).bool())
    o, lse = ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qunion, sm, plan.qpair, plan.qorder)
    plan.build_key_lists()
    monkeypatch.setenv("PRISM_DEBUG", "1")
    say("debug: valid lists")
    o2, lse2 = ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qunion, sm, plan.qpair, plan.qorder)
    assert bits_equal(host(o), host(o2)) and bits_equal(host(lse), host(lse2))
    us, ul, uc = plan.qunion
    r = int(torch.nonzero(ul >= 2)[0, 0])
    s = int(us[r])
    bad = uc.clone()
    bad[s], bad[s + 1] = uc[s + 1], uc[s]
    say("debug: descending union entries")
    with pytest.raises(ValueError, match="not above"):
        ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, (us, ul, bad), sm, plan.qpair, plan.qorder)
    bad_order = plan.qorder.clone()
    bad_order[1] = bad_order[0]
    say("debug: launch order with a repeated pair")
    with pytest.raises(ValueError, match="twice"):
        ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qunion, sm, plan.qpair, bad_order)
    ks, kl, kc = plan.kunion
    bad_k = kc.clone()
    bad_k[int(ks[int(torch.nonzero(kl >= 1)[0, 0])])] |= 4  # a partial flag on a query-tile list
    rng = np.random.default_rng(5)
    do_t = dev(bf16(rng.standard_normal((B, H, S, D)).astype(np.float32)))
    delta = ops.bwd_preprocess(o, do_t)
    m2 = ops.lse_to_m2(lse)
    say("debug: partial flag in a dK/dV list")
    with pytest.raises(ValueError, match="flagged partial"):
        ops.bsa_bwd(plan.q_re, plan.k_re, plan.v_re, do_t, m2, delta, plan.kv_valid, plan.tmasks, plan.qunion,
                    (ks, kl, bad_k), sm, plan.qpair, plan.kpair, plan.qorder, plan.korder)
    torch.cuda.synchronize()


def test_work_queue_bit_identical(case):
    """The attention entry points through the C-ABI with work_counter = NULL
    (one workgroup per pair) and with a counter (persistent workgroups taking
    pairs from a work queue; the counter starts with garbage, which the call
    clears, and is reused by the next call) give the same bits as the
    operators, which always pass a counter."""
    from prism_amd import ops, plan_dynamic
    valid = case["valid"] if case["pad"] else None
    B, H, S, D = case["q"].shape
    BH, sm = B * H, 1 / math.sqrt(D)
    plan = plan_dynamic(dev(case["qh"]), dev(case["kh"]), dev(case["vh"]), case["grid"], method="ivpq",
                        sparsity=0.6, cdf_threshold=0.9, valid_mask=None if valid is None else dev(valid).bool())
    ptr = lambda t: None if t is None else t.data_ptr()
    stream = torch.cuda.current_stream().cuda_stream
    qorder = ops.pair_order(plan.qunion[1], 64)
    o, lse = ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qunion, sm, plan.qpair, qorder)
    counter = torch.full((8,), 12345, dtype=torch.int32, device="cuda")
    for ctr in (None, counter, counter):
        say("work queue: forward, counter", ctr is not None)
        o2, lse2 = torch.empty_like(o), torch.empty_like(lse)
        ops._lib.call("prism_bsa_fwd", ptr(plan.q_re), ptr(plan.k_re), ptr(plan.v_re), BH, S, S, D, ptr(plan.tmasks),
                      *(ptr(t) for t in plan.qunion), ptr(plan.qpair), ptr(qorder), sm, ptr(o2), ptr(lse2), ptr(ctr),
                      stream)
        assert bits_equal(host(o), host(o2)) and bits_equal(host(lse), host(lse2))
    rng = np.random.default_rng(98)
    do_t = dev(bf16(rng.standard_normal((B, H, S, D)).astype(np.float32)))
    delta = ops.bwd_preprocess(o, do_t)
    m2 = ops.lse_to_m2(lse)
    klists = ops.transpose_lists(plan.qstart, plan.qlen, plan.qcols, BH, plan.lay.Nt)
    kpair = ops.pair_tiles(*klists, plan.lay.Nt)
    kunion = ops.pair_union(*klists, plan.lay.Nt, pairmap=kpair)
    korder = ops.pair_order(kunion[1], 32)
    dq, dk, dv = ops.bsa_bwd(plan.q_re, plan.k_re, plan.v_re, do_t, m2, delta, plan.kv_valid, plan.tmasks,
                             plan.qunion, kunion, sm, plan.qpair, kpair, qorder, korder)
    common = (ptr(plan.q_re), ptr(plan.k_re), ptr(plan.v_re), ptr(do_t), ptr(m2), ptr(delta), BH, S, S, D)
    for ctr in (None, counter, counter):
        say("work queue: backward, counter", ctr is not None)
        dk2, dv2, dq2 = torch.empty_like(dk), torch.empty_like(dv), torch.empty_like(dq)
        counter.fill_(-7)
        ops._lib.call("prism_bsa_bwd_dkdv", *common, ptr(plan.kv_valid), *(ptr(t) for t in kunion), ptr(kpair),
                      ptr(korder), sm, ptr(dk2), ptr(dv2), ptr(ctr), stream)
        ops._lib.call("prism_bsa_bwd_dq", *common, ptr(plan.tmasks), *(ptr(t) for t in plan.qunion), ptr(plan.qpair),
                      ptr(qorder), sm, ptr(dq2), ptr(ctr), stream)
        for g, g2 in ((dq, dq2), (dk, dk2), (dv, dv2)):
            assert bits_equal(host(g), host(g2))


def test_attention_graph_capture_replays(case):
    """Forward and backward over a prebuilt plan, captured in one HIP graph
    (persistent launches with their counter-zeroing kernels, the operators'
    outputs and counters from the graph's memory pool): three replays, with
    eager work and synchronisations between them, each give the eager bits."""
    from prism_amd import ops, plan_dynamic
    valid = case["valid"] if case["pad"] else None
    B, H, S, D = case["q"].shape
    sm = 1 / math.sqrt(D)
    plan = plan_dynamic(dev(case["qh"]), dev(case["kh"]), dev(case["vh"]), case["grid"], method="ivpq",
                        sparsity=0.6, cdf_threshold=0.9, valid_mask=None if valid is None else dev(valid).bool())
    rng = np.random.default_rng(97)
    do_t = dev(bf16(rng.standard_normal((B, H, S, D)).astype(np.float32)))
    qorder = ops.pair_order(plan.qunion[1], 64)
    klists = ops.transpose_lists(plan.qstart, plan.qlen, plan.qcols, B * H, plan.lay.Nt)
    kpair = ops.pair_tiles(*klists, plan.lay.Nt)
    kunion = ops.pair_union(*klists, plan.lay.Nt, pairmap=kpair)
    korder = ops.pair_order(kunion[1], 32)

    def step():
        o, lse = ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qunion, sm, plan.qpair, qorder)
        delta = ops.bwd_preprocess(o, do_t)
        dq, dk, dv = ops.bsa_bwd(plan.q_re, plan.k_re, plan.v_re, do_t, ops.lse_to_m2(lse), delta, plan.kv_valid,
                                 plan.tmasks, plan.qunion, kunion, sm, plan.qpair, kpair, qorder, korder)
        return o, lse, dq, dk, dv

    ref = [host(t) for t in step()]
    warm = torch.cuda.Stream()
    warm.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(warm):
        step()
    torch.cuda.current_stream().wait_stream(warm)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    for rep in range(3):
        say("graph replay", rep)
        junk = torch.full((1 << 20,), float(rep), device="cuda").cumsum(0)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, t, r in zip(("O", "LSE", "dQ", "dK", "dV"), outs, ref):
            assert bits_equal(host(t), r), (rep, name)
        del junk


@pytest.mark.parametrize("compute_padded", [False, True, None])
def test_end_to_end_autograd(case, compute_padded):
    """flash_attn_bsa_3d_dynamic forward + backward through autograd in THW
    order vs the oracle attention on the oracle's own selection (with and
    without attention for fully padded query tiles; None = the default call,
    which attends for them as the reference does)."""
    from prism_amd import flash_attn_bsa_3d_dynamic
    valid = case["valid"] if case["pad"] else None
    B, H, S, D = case["q"].shape
    sm = 1 / math.sqrt(D)
    ref = O.select_pipeline(case["qh"], case["kh"], case["vh"], case["grid"], method="ivpq", sparsity=0.7,
                            cdf_threshold_p=0.9, audio_norms=case["nh"], valid=valid,
                            skip_padded_queries=compute_padded is False)
    src, inv = O.rearrange_index(ref["shape_ids"], case["grid"])
    tof = (lambda a: O.bf16_bits_to_f32(a)) if case["qh"].dtype == np.uint16 else (lambda a: O.bf16_bits_to_f32(bf16(a)))
    qf, kf, vf = (tof(case[n])[:, :, src].reshape(B * H, S, D) for n in ("qh", "kh", "vh"))
    kv = None if valid is None else valid[src]
    o_ref, lse_ref = O.attn_fwd(qf, kf, vf, ref["qstart"], ref["qlen"], ref["qcols"], kv, sm)
    tdt = torch.bfloat16 if case["qh"].dtype == np.uint16 else torch.float32
    q, k, v = (dev(case[n]).requires_grad_(True) for n in ("qh", "kh", "vh"))
    kw = {} if compute_padded is None else {"compute_padded_queries": compute_padded}
    out, sid = flash_attn_bsa_3d_dynamic(q, k, v, case["grid"], method="ivpq", sparsity=0.7, cdf_threshold=0.9,
                                         audio_token_norms=None if case["nh"] is None else dev(case["nh"]),
                                         valid_mask=None if valid is None else dev(valid).bool(),
                                         return_shape_ids=True, **kw)
    assert out.dtype == tdt
    assert np.array_equal(host(sid), ref["shape_ids"])
    og = out.detach().float().cpu().numpy().reshape(B * H, S, D)
    _tol(og, o_ref[:, inv], "O(THW)")
    rng = np.random.default_rng(3)
    do = rng.standard_normal((B, H, S, D)).astype(np.float32)
    do_q = O.bf16_bits_to_f32(bf16(do))
    out.backward(torch.from_numpy(do_q).to(DEV).to(tdt))
    o_bf = O.bf16_bits_to_f32(bf16(o_ref.astype(np.float32)))
    dq_r, dk_r, dv_r = O.attn_bwd(qf, kf, vf, o_bf, do_q.reshape(B * H, S, D)[:, src], lse_ref, ref["qstart"],
                                  ref["qlen"], ref["qcols"], kv, sm)
    for name, t, r in (("dQ", q, dq_r), ("dK", k, dk_r), ("dV", v, dv_r)):
        _tol(t.grad.float().cpu().numpy().reshape(B * H, S, D), r[:, inv], name + "(THW)")


def test_determinism(case):
    """Two identical calls give bit-identical outputs and gradients."""
    from prism_amd import flash_attn_bsa_3d_dynamic
    valid = case["valid"] if case["pad"] else None
    outs = []
    for _ in range(2):
        q, k, v = (dev(case[n]).requires_grad_(True) for n in ("qh", "kh", "vh"))
        o = flash_attn_bsa_3d_dynamic(q, k, v, case["grid"], method="penalty", sparsity=0.5, cdf_threshold=0.9,
                                      valid_mask=None if valid is None else dev(valid).bool())
        o.backward(torch.ones_like(o))
        outs.append([host(o), host(q.grad), host(k.grad), host(v.grad)])
    for a, b in zip(*outs):
        assert np.array_equal(a, b)
