"""Pin the oracle's geometry, pooling, scores, selection and list functions
against independent formulations: numpy reshape/transpose geometry, float64
means and matmuls, stable-sort top-k, a float64 nucleus (top-p) selection, the
reference's own torch-op sequence for the selection helpers
(bsa_interface.py:235-304) evaluated with torch on the CPU, and brute-force
set transposes.  CPU only.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.cases import bf16

CAND = O.CANDIDATES


# ------------------------------------------------------------------ geometry (a8)
def _np_zone_order(shape):
    """Local flat coordinates (lt*64 + lh*8 + lw) in rearranged order for one
    zone, built by reshape/transpose: blocks t-major then h then w, tokens
    inside a block t-major then h then w."""
    bt, bh, bw = shape
    lf = np.arange(512).reshape(8, 8, 8)
    x = lf.reshape(8 // bt, bt, 8 // bh, bh, 8 // bw, bw).transpose(0, 2, 4, 1, 3, 5)
    return x.reshape(-1)


@pytest.mark.parametrize("grid", [(8, 8, 8), (16, 24, 8), (8, 16, 32)])
def test_rearrange_index_matches_reshape_transpose(grid):
    T, Hg, Wg = grid
    ZT, ZH, ZW = T // 8, Hg // 8, Wg // 8
    Nz = ZT * ZH * ZW
    rng = np.random.default_rng(sum(grid))
    sid = rng.integers(0, 13, Nz)
    sid[: min(Nz, 13)] = np.arange(min(Nz, 13))
    src, inv = O.rearrange_index(sid, grid)
    thw = np.arange(T * Hg * Wg).reshape(T, Hg, Wg)
    for z in range(Nz):
        zt, zh, zw = z // (ZH * ZW), (z // ZW) % ZH, z % ZW
        box = thw[zt * 8:(zt + 1) * 8, zh * 8:(zh + 1) * 8, zw * 8:(zw + 1) * 8].reshape(-1)
        assert np.array_equal(src[z * 512:(z + 1) * 512], box[_np_zone_order(CAND[sid[z]])])
    assert np.array_equal(np.sort(src), np.arange(T * Hg * Wg))  # a permutation
    assert np.array_equal(inv[src], np.arange(T * Hg * Wg))      # and its inverse


def test_every_block_is_a_subbox_of_its_shape():
    for c, (bt, bh, bw) in enumerate(CAND):
        order = np.array([O.lib().oc_local_of_rearr(c, r) for r in range(512)])
        bsz = bt * bh * bw
        for b in range(512 // bsz):
            lf = order[b * bsz:(b + 1) * bsz]
            lt, lh, lw = lf // 64, (lf // 8) % 8, lf % 8
            assert (lt.max() - lt.min() + 1, lh.max() - lh.min() + 1, lw.max() - lw.min() + 1) == (bt, bh, bw)
            assert len(set(lf.tolist())) == bsz


def test_tile_maps_brute_force():
    rng = np.random.default_rng(3)
    sid = rng.integers(0, 13, 40)
    bot, kbt, nb, boff = O.tile_maps(sid)
    Nt = 40 * 8
    exp_bot, exp_kbt, exp_off, b = [], [], [], 0
    for z, c in enumerate(sid):
        tpb = int(np.prod(CAND[c])) // 64
        exp_off.append(b)
        for j in range(8 // tpb):
            tiles = [z * 8 + j * tpb + i for i in range(tpb)]
            exp_kbt.append(tiles + [Nt] * (2 - tpb))
            exp_bot += [b] * tpb
            b += 1
    exp_kbt.append([Nt, Nt])
    assert nb == b
    assert np.array_equal(bot, exp_bot) and np.array_equal(boff, exp_off)
    assert np.array_equal(kbt, np.array(exp_kbt))


# ------------------------------------------------------------------ pooling and scores (a10, a11)
def test_block_pool_vs_float64_masked_means():
    rng = np.random.default_rng(4)
    grid = (8, 16, 16)
    S = 8 * 16 * 16
    x = rng.standard_normal((2, 3, S, 64)).astype(np.float32)
    valid = (rng.random(S) > 0.3).astype(np.uint8)
    valid.reshape(8, 16, 16)[:, :8, :8] = 0  # zone 0 fully padded
    sid = np.array([0, 7, 12, 3])
    out, bc, tc = O.block_pool(x, sid, grid, valid)
    src, _ = O.rearrange_index(sid, grid)
    xr = x[:, :, src].astype(np.float64)
    vr = valid[src].astype(bool)
    b = 0
    for z, c in enumerate(sid):
        bsz = int(np.prod(CAND[c]))
        for j in range(512 // bsz):
            sl = slice(z * 512 + j * bsz, z * 512 + (j + 1) * bsz)
            m = vr[sl]
            assert bc[b] == m.sum()
            ref = xr[:, :, sl][:, :, m].sum(2) / max(m.sum(), 1)
            assert np.allclose(out[:, :, b], ref, rtol=1e-5, atol=1e-6)
            b += 1
    assert np.array_equal(tc, vr.reshape(-1, 64).sum(1))
    assert np.all(out[:, :, :8] == 0)


def test_block_scores_exact_on_integers_and_close_on_floats():
    rng = np.random.default_rng(5)
    qi = rng.integers(-20, 20, (2, 50, 64)).astype(np.float32)
    ki = rng.integers(-20, 20, (2, 50, 64)).astype(np.float32)
    bc = np.ones(50, np.int32)
    bc[[3, 17]] = 0
    s = O.block_scores(qi, ki, bc)
    ref = np.einsum("bnd,bmd->bnm", qi.astype(np.int64), ki.astype(np.int64)).astype(np.float32)
    ref[:, :, [3, 17]] = -np.inf
    assert np.array_equal(s, ref)
    qf = rng.standard_normal((1, 40, 128)).astype(np.float32)
    kf = rng.standard_normal((1, 40, 128)).astype(np.float32)
    s = O.block_scores(qf, kf, None)
    assert np.allclose(s, qf.astype(np.float64) @ kf.astype(np.float64).transpose(0, 2, 1), atol=1e-4)


# ------------------------------------------------------------------ selection (a12)
def _scores(rng, rows, N, kind):
    s = rng.standard_normal((rows, N)).astype(np.float32) * 3
    if kind == "ties":
        s = np.round(s * 2) / 2
    elif kind == "neginf":
        s[:, rng.random(N) < 0.2] = -np.inf
    elif kind == "peaked":
        s[:, : max(1, N // 10)] += 8
    return s


@pytest.mark.parametrize("kind", ["plain", "ties", "neginf"])
def test_topk_is_stable_sort_topk(kind):
    """Mode 0: the k largest scores, ties to the lower index (a total order
    that the reference's torch.topk leaves unspecified)."""
    rng = np.random.default_rng(6)
    for N in (17, 200, 1000):
        s = _scores(rng, 16, N, kind)
        for sp in (0.9, 0.5, 0.01):
            k = int((1 - sp) * N)
            sel, n = O.select(s, sp, None, 0.125)
            assert np.all(n == k)
            for r in range(len(s)):
                order = np.lexsort((np.arange(N), -s[r].astype(np.float64)))
                assert np.array_equal(sel[r, :k], np.sort(order[:k]))


def _nucleus64(s, sparsity, p, scale):
    """float64 nucleus selection: returns (set, margin) where margin is the
    distance of the cumulative sum at the decision from p (ties across the
    boundary give margin 0)."""
    N = s.shape[0]
    x = s.astype(np.float64) * np.float64(np.float32(scale))
    if not np.isfinite(x).any():
        return set(), np.inf
    w = np.exp(x - x.max())
    w /= w.sum()
    order = np.lexsort((np.arange(N), -w))
    mode, k_lo, ub = O.selection_params(N, sparsity, p)
    cdf = np.cumsum(w[order][:ub])
    c = int((cdf < p).sum())
    n = min(max(c + 1, k_lo), N)
    eff = min(n, ub)
    margin = np.abs(cdf - p).min()
    ws = w[order]
    if eff < N and ws[eff - 1] - ws[eff] < 1e-12:
        margin = 0.0
    return set(order[:eff].tolist()), margin


@pytest.mark.parametrize("kind", ["plain", "neginf", "peaked"])
@pytest.mark.parametrize("params", [(None, 0.9), (None, 0.2), (0.95, 0.9), (0.5, 0.3)])
def test_nucleus_selection_vs_float64(kind, params):
    """Modes 1 and 2 agree with an exact (float64) nucleus selection on every
    row whose decision is farther than 1e-5 from the threshold."""
    sp, p = params
    rng = np.random.default_rng(7)
    checked = 0
    for N in (30, 300, 2000):
        s = _scores(rng, 24, N, kind)
        sel, n = O.select(s, sp, p, 0.125)
        for r in range(len(s)):
            ref, margin = _nucleus64(s[r], sp, p, 0.125)
            if margin < 1e-5:
                continue
            checked += 1
            assert set(sel[r, : n[r]].tolist()) == ref, (N, r)
            assert np.all(np.diff(sel[r, : n[r]]) > 0)
    assert checked >= 40


def _torch_reference_select(score, sparsity, p, sm_scale):
    """The reference's selection helpers (bsa_interface.py:235-304), the same
    torch op sequence evaluated on the CPU in float32: returns per-row sets,
    per-row decision margins |cdf - p| and "tie at the boundary" flags."""
    score = torch.from_numpy(score)
    Sk = score.shape[-1]
    if p is None:
        k = int((1 - sparsity) * Sk)
        vals, idx = torch.topk(score, k)
        sets = [set(r.tolist()) for r in idx]
        srt = torch.sort(score, dim=-1, descending=True).values
        tie = (srt[:, k - 1] == srt[:, k]) if k < Sk else torch.zeros(len(score), dtype=torch.bool)
        return sets, torch.full((len(score),), float("inf")), tie
    weights = torch.softmax(score * sm_scale, dim=-1)
    lo = 1 if sparsity is None else max(1, int((1 - sparsity) * Sk))
    ub = min(Sk, max(lo, int(p * Sk) + 1))
    vals, idx = torch.topk(weights, k=ub, dim=-1, largest=True, sorted=True)
    cdf = torch.cumsum(vals, dim=-1)
    n = ((cdf < p).to(torch.int32).sum(dim=-1, keepdim=True) + 1).clamp(min=lo, max=Sk)
    pos = torch.arange(ub)
    idx = idx.masked_fill(pos >= n, Sk)
    sets = [set(x for x in r.tolist() if x < Sk) for r in idx]
    # decision margin: distance from p of the exact (float64) cumulative sums
    # of the float32 weights on either side of the crossing
    c = (cdf < p).to(torch.int64).sum(dim=-1)  # crossing position (== ub when never crossed)
    cdf64 = torch.cumsum(vals.double(), dim=-1)
    near = torch.stack([(cdf64.gather(1, (c - d).clamp(0, ub - 1)[:, None])[:, 0] - p).abs() for d in (0, 1)])
    margin = near.min(dim=0).values
    srt = torch.sort(weights, dim=-1, descending=True).values
    e = torch.clamp(n.squeeze(-1), max=ub)
    tie = torch.tensor([bool(e[i] < Sk and srt[i, e[i] - 1] == srt[i, e[i]]) for i in range(len(score))])
    return sets, margin, tie


@pytest.mark.parametrize("params", [(0.9, None), (None, 0.9), (0.97, 0.9), (0.75, 0.5)])
def test_selection_agrees_with_reference_torch_semantics(params):
    """Same fp32 scores -> same selected set as the reference's torch op
    sequence, on every row not decided within float32 rounding of p (those
    rows are counted and must be rare)."""
    sp, p = params
    rng = np.random.default_rng(8)
    total = agree = skipped = 0
    for N in (64, 720, 1500):
        s = _scores(rng, 32, N, "peaked" if N == 720 else "plain")
        sel, n = O.select(s, sp, p, 1 / math.sqrt(128))
        sets, margin, tie = _torch_reference_select(s, sp, p, 1 / math.sqrt(128))
        for r in range(len(s)):
            total += 1
            if bool(tie[r]) or float(margin[r]) < 1e-6:
                skipped += 1
                continue
            assert set(sel[r, : n[r]].tolist()) == sets[r], (N, r)
            agree += 1
    assert skipped <= total // 10, (skipped, total)
    assert agree >= total - skipped


def test_planted_mistakes_fail():
    """The float64 / torch checks above catch the plausible mistakes: a
    nucleus without the crossing block, and <= instead of < at the threshold."""
    rng = np.random.default_rng(9)
    s = _scores(rng, 16, 400, "plain")
    sel, n = O.select(s, None, 0.9, 0.125)
    diffs = 0
    for r in range(len(s)):
        ref, margin = _nucleus64(s[r], None, 0.9, 0.125)
        if margin < 1e-5:
            continue
        wrong = set(sel[r, : n[r] - 1].tolist())  # crossing block dropped
        diffs += wrong != ref
    assert diffs > 10


def test_all_neginf_row_selects_nothing_in_cdf_mode():
    s = np.full((2, 50), -np.inf, np.float32)
    sel, n = O.select(s, None, 0.9, 0.1)
    assert np.all(n == 0)
    sel, n = O.select(s, 0.5, None, 0.1)  # top-k still picks k (all -inf), as torch.topk does
    assert np.all(n == 25)


# ------------------------------------------------------------------ expansion and transpose (a13, a15)
def test_expand_tiles_brute_force():
    rng = np.random.default_rng(10)
    sid = rng.integers(0, 13, 12)
    bot, kbt, nb, _ = O.tile_maps(sid)
    Nt = 12 * 8
    tile_count = rng.integers(0, 3, Nt).astype(np.int32)
    cap = 10
    sel = np.full((nb, cap), -1, np.int64)
    nsel = rng.integers(0, cap + 1, nb).astype(np.int32)
    for r in range(nb):
        sel[r, : nsel[r]] = np.sort(rng.choice(nb, nsel[r], replace=False))
    tiles, nt = O.expand_tiles(sel, nsel, kbt, Nt, tile_count)
    for r in range(nb):
        exp = sorted(t for b in sel[r, : nsel[r]] for t in kbt[b] if t < Nt and tile_count[t] > 0)
        assert tiles[r, : nt[r]].tolist() == exp


def test_transpose_lists_brute_force():
    rng = np.random.default_rng(11)
    BH, Nt = 2, 40
    cap = 12
    qlen = rng.integers(0, cap + 1, BH * Nt).astype(np.int32)
    qcols = np.zeros(BH * Nt * cap, np.int32)
    for r in range(BH * Nt):
        qcols[r * cap: r * cap + qlen[r]] = np.sort(rng.choice(Nt, qlen[r], replace=False))
    qstart = np.arange(BH * Nt, dtype=np.int64) * cap
    kcols, klen = O.transpose_lists(qstart, qlen, qcols, BH, Nt)
    for bh in range(BH):
        for kt in range(Nt):
            exp = [t for t in range(Nt) if kt in set(qcols[(bh * Nt + t) * cap:(bh * Nt + t) * cap + qlen[bh * Nt + t]])]
            row = bh * Nt + kt
            assert kcols[row, : klen[row]].tolist() == exp


# ------------------------------------------------------------------ whole selection path vs the reference's torch steps
def test_select_pipeline_vs_reference_torch_steps():
    """Steps (2)-(5) of flash_attn_bsa_3d_dynamic (dynamic_block_attention.py:243-319)
    restated with torch ops on the CPU in float32 from the oracle's shape ids:
    gather, masked tile means, count-weighted block means, scores with
    invalid keys at -inf, hybrid selection, tile expansion.  Tile lists must
    agree on every row not decided within rounding of the threshold."""
    from tests.cases import padded_case
    c = padded_case(0, 1, 2, (5, 12, 16), 64)
    grid = c["grid"]
    B, H, S, D = c["q"].shape
    sp, p = 0.8, 0.9
    sm = 1 / math.sqrt(D)
    ref = O.select_pipeline(c["q"], c["k"], c["v"], grid, sparsity=sp, cdf_threshold_p=p, valid=c["valid"])
    sid = ref["shape_ids"]
    src, _ = O.rearrange_index(sid, grid)
    bot, kbt, nb, _ = O.tile_maps(sid)
    Nt = S // 64
    valid_re = torch.from_numpy(c["valid"][src].astype(bool))
    q_re = torch.from_numpy(c["q"][:, :, src])
    k_re = torch.from_numpy(c["k"][:, :, src])

    def tile_means(x):
        m = valid_re.view(Nt, 64).float()[None, None, :, :, None]
        return (x.view(B, H, Nt, 64, D) * m).sum(3) / m.sum(3).clamp(min=1.0)

    tc = valid_re.view(Nt, 64).sum(-1).float()
    bidx = torch.from_numpy(bot)

    def block_means(xt):
        bs = xt.new_zeros(B, H, nb, D).index_add_(2, bidx, xt * tc.view(1, 1, Nt, 1))
        cnt = tc.new_zeros(nb).index_add_(0, bidx, tc)
        return bs / cnt.clamp(min=1.0).view(1, 1, nb, 1), cnt

    qc, _ = block_means(tile_means(q_re))
    kc, cnt = block_means(tile_means(k_re))
    score = (qc @ kc.transpose(-1, -2)).masked_fill((cnt == 0).view(1, 1, 1, -1), float("-inf"))
    sets, margin, tie = _torch_reference_select(score.reshape(B * H * nb, nb).numpy(), sp, p, sm)
    tcnt = tc.numpy()
    checked = 0
    for r in range(B * H * nb):
        if bool(tie[r]) or float(margin[r]) < 1e-4:
            continue
        exp = sorted(t for b in sets[r] for t in kbt[b] if t < Nt and tcnt[t] > 0)
        assert ref["tiles"][r, : ref["ntiles"][r]].tolist() == exp, r
        checked += 1
    assert checked >= (B * H * nb) * 3 // 4


def test_skip_padded_queries_only_empties_fully_padded_tiles():
    from tests.cases import padded_case
    c = padded_case(1, 1, 1, (5, 12, 16), 64)
    full = O.select_pipeline(c["q"], c["k"], c["v"], c["grid"], sparsity=0.8, cdf_threshold_p=0.9, valid=c["valid"])
    skip = O.select_pipeline(c["q"], c["k"], c["v"], c["grid"], sparsity=0.8, cdf_threshold_p=0.9, valid=c["valid"],
                             skip_padded_queries=True)
    empty = full["tile_count"] == 0
    assert empty.any() and (~empty).any()
    assert np.all(skip["qlen"][empty] == 0)
    assert np.array_equal(skip["qlen"][~empty], full["qlen"][~empty])


def test_pair_union_brute_force():
    """oracle.pair_union vs Python set arithmetic on random sorted lists
    (empty rows, identical rows, disjoint rows) and tile masks."""
    rng = np.random.default_rng(5)
    Nt, rows = 40, 12
    lists = []
    for r in range(rows):
        kind = r % 4
        if kind == 0:
            lists.append([])
        elif kind == 1 and r > 0:
            lists.append(list(lists[-1]))
        else:
            lists.append(sorted(rng.choice(Nt, size=int(rng.integers(1, Nt)), replace=False).tolist()))
    cap = Nt
    start = np.arange(rows, dtype=np.int64) * cap
    length = np.array([len(x) for x in lists], np.int32)
    cols = np.full(rows * cap, -7, np.int32)
    for r, x in enumerate(lists):
        cols[r * cap: r * cap + len(x)] = x
    valid = (rng.random(Nt * O.TILE) > 0.02).astype(np.uint8)
    valid[: 5 * O.TILE] = 1
    masks = O.tile_masks(valid)
    for t in range(Nt):
        want = sum(1 << j for j in range(O.TILE) if valid[t * O.TILE + j])
        assert int(masks[t]) == want
    got = O.pair_union(start, length, cols, Nt, masks)
    assert len(got) == rows // 2
    for p in range(rows // 2):
        a, b = set(lists[2 * p]), set(lists[2 * p + 1])
        want = []
        for t in sorted(a | b):
            partial = int(masks[t]) != (1 << 64) - 1
            want.append(t * 8 + (4 if partial else 0) + (2 if t in b else 0) + (1 if t in a else 0))
        assert got[p].tolist() == want


def _all_matchings(items):
    """Every perfect matching of `items` (independent enumeration)."""
    if not items:
        yield []
        return
    first, rest = items[0], items[1:]
    for i, b in enumerate(rest):
        for m in _all_matchings(rest[:i] + rest[i + 1:]):
            yield [(first, b)] + m


def test_pair_tiles_brute_force():
    """The pairing of each group of 8 tiles (6 at the end of a head of 14)
    has the largest summed list overlap of all perfect matchings; identical
    lists (all matchings tie) pair neighbours."""
    rng = np.random.default_rng(31)
    Nt, BH, ncols = 14, 2, 40
    rows = BH * Nt
    lists = [sorted(rng.choice(ncols, size=int(rng.integers(0, ncols)), replace=False).tolist()) for _ in range(rows)]
    cap = ncols
    start = np.arange(rows, dtype=np.int64) * cap
    length = np.array([len(x) for x in lists], np.int32)
    cols = np.full(rows * cap, -1, np.int32)
    for r, x in enumerate(lists):
        cols[r * cap: r * cap + len(x)] = x
    pm = O.pair_tiles(start, length, cols, Nt, ncols)
    for h in range(BH):
        for r0, g in ((0, 8), (8, 6)):
            got = [(int(pm[h * Nt + r0 + 2 * k]) - r0, int(pm[h * Nt + r0 + 2 * k + 1]) - r0) for k in range(g // 2)]
            assert sorted(a for p in got for a in p) == list(range(g))       # a perfect matching of the group
            assert all(a < b for a, b in got) and [a for a, _ in got] == sorted(a for a, _ in got)
            sets = [set(lists[h * Nt + r0 + i]) for i in range(g)]
            score = lambda m: sum(len(sets[a] & sets[b]) for a, b in m)
            assert score(got) == max(score(m) for m in _all_matchings(list(range(g))))
    # all lists equal: every matching ties, the first (neighbours) is taken
    same = O.pair_tiles(np.zeros(8, np.int64), np.full(8, 3, np.int32), np.array([1, 2, 3], np.int32), 8, 4)
    assert same.tolist() == list(range(8))
    # paired unions use the pairmap's rows
    u = O.pair_union(start, length, cols, Nt, None, pm)
    for p in range(rows // 2):
        h0 = (2 * p) // Nt * Nt
        a, b = h0 + pm[2 * p], h0 + pm[2 * p + 1]
        assert (u[p] >> 3).tolist() == sorted(set(lists[a]) | set(lists[b]))
