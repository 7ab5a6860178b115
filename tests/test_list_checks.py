"""The work-list checks of the debug mode (prism_check_lists,
prism_check_launch_maps; host memory, no GPU): valid lists pass, and each
kind of corruption the attention kernels could not survive is rejected with
ValueError before anything is launched."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from prism_amd import _lib

NT = 48      # tiles per head
HEADS = 2


def ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def check_lists(start, length, cols, ntiles, unions, masks=None):
    start = np.ascontiguousarray(start, np.int64)
    length = np.ascontiguousarray(length, np.int32)
    cols = np.ascontiguousarray(cols, np.int32)
    masks = None if masks is None else np.ascontiguousarray(masks, np.uint64)
    _lib.call("prism_check_lists", ptr(start), ptr(length), ptr(cols), start.size, cols.size, ntiles, int(unions),
              ptr(masks))


def check_maps(pairmap, heads, tiles, order):
    pairmap = None if pairmap is None else np.ascontiguousarray(pairmap, np.int32)
    order = None if order is None else np.ascontiguousarray(order, np.int32)
    _lib.call("prism_check_launch_maps", ptr(pairmap), heads, tiles, ptr(order), 0 if order is None else order.size)


@pytest.fixture(scope="module")
def lists():
    """Dense-compat per-query-tile lists (start = row * cap) of two heads, the
    key mask of a padded last tile, their pairing and pair unions as the
    kernels take them."""
    rng = np.random.default_rng(3)
    rows, cap = HEADS * NT, NT
    start = np.arange(rows, dtype=np.int64) * cap
    length = rng.integers(0, NT + 1, rows).astype(np.int32)
    cols = np.full(rows * cap, -1, np.int32)
    for r in range(rows):
        cols[start[r]: start[r] + length[r]] = np.sort(rng.choice(NT, length[r], replace=False))
    valid = np.ones(NT * 64, np.uint8)
    valid[-20:] = 0
    masks = O.tile_masks(valid)
    pairmap = O.pair_tiles(start, length, cols, NT)
    unions = O.pair_union(start, length, cols, NT, masks, pairmap)
    ustart = np.arange(len(unions), dtype=np.int64) * NT
    ulen = np.array([len(u) for u in unions], np.int32)
    ucols = np.zeros(len(unions) * NT, np.int32)
    for p, u in enumerate(unions):
        ucols[ustart[p]: ustart[p] + len(u)] = u
    order = np.random.default_rng(4).permutation(len(unions)).astype(np.int32)
    return dict(start=start, length=length, cols=cols, masks=masks, pairmap=pairmap, ustart=ustart, ulen=ulen,
                ucols=ucols, order=order)


def test_valid_lists_pass(lists):
    L = lists
    check_lists(L["start"], L["length"], L["cols"], NT, False)
    check_lists(L["ustart"], L["ulen"], L["ucols"], NT, True, L["masks"])
    check_maps(L["pairmap"], HEADS, NT, L["order"])
    check_maps(None, HEADS, NT, None)
    # unions built without masks carry no partial flags
    u = O.pair_union(L["start"], L["length"], L["cols"], NT, None, L["pairmap"])
    us = np.cumsum([0] + [len(x) for x in u])[:-1]
    check_lists(us, [len(x) for x in u], np.concatenate(u), NT, True, None)


def _first_row(length, at_least=2):
    return int(np.nonzero(np.asarray(length) >= at_least)[0][0])


@pytest.mark.parametrize("kind", ["tile_out_of_range", "negative_tile", "descending", "duplicate", "past_entries",
                                  "negative_start", "negative_length", "length_over_tiles"])
def test_corrupt_plain_lists_raise(lists, kind):
    L = lists
    start, length, cols = L["start"].copy(), L["length"].copy(), L["cols"].copy()
    r = _first_row(length)
    s = int(start[r])
    match = {"tile_out_of_range": "outside \\[0", "negative_tile": "outside \\[0", "descending": "not above",
             "duplicate": "not above", "past_entries": "outside the", "negative_start": "outside the",
             "negative_length": "length", "length_over_tiles": "length"}[kind]
    if kind == "tile_out_of_range":
        cols[s + length[r] - 1] = NT
    elif kind == "negative_tile":
        cols[s] = -1
    elif kind == "descending":
        cols[s], cols[s + 1] = cols[s + 1], cols[s]
    elif kind == "duplicate":
        cols[s + 1] = cols[s]
    elif kind == "past_entries":
        start[-1] = cols.size - length[-1] + 1 if length[-1] else cols.size + 1
        length[-1] = max(int(length[-1]), 1)
    elif kind == "negative_start":
        start[r] = -1
    elif kind == "negative_length":
        length[r] = -1
    else:
        length[r] = NT + 1
    with pytest.raises(ValueError, match=match):
        check_lists(start, length, cols, NT, False)


@pytest.mark.parametrize("kind", ["no_member_flag", "partial_flag_missing", "partial_flag_spurious",
                                  "partial_without_masks", "tile_out_of_range"])
def test_corrupt_unions_raise(lists, kind):
    L = lists
    ustart, ulen, ucols = L["ustart"], L["ulen"], L["ucols"].copy()
    masks = L["masks"]
    last = NT - 1  # the padded tile
    hits = [(p, i) for p in range(ulen.size) for i in range(ulen[p]) if ucols[ustart[p] + i] >> 3 == last]
    full = [(p, i) for p in range(ulen.size) for i in range(ulen[p]) if ucols[ustart[p] + i] >> 3 != last]
    if kind == "no_member_flag":
        p, i = full[0]
        ucols[ustart[p] + i] &= ~3
        match = "belongs to no tile"
    elif kind == "partial_flag_missing":
        p, i = hits[0]
        ucols[ustart[p] + i] &= ~4
        match = "flagged full but its key mask is partial"
    elif kind == "partial_flag_spurious":
        p, i = full[0]
        ucols[ustart[p] + i] |= 4
        match = "flagged partial but its key mask is full"
    elif kind == "partial_without_masks":
        masks = None
        match = "flagged partial but its key mask is absent"
    else:
        p, i = hits[0]
        ucols[ustart[p] + i] = (NT << 3) | 1
        match = "outside \\[0"
    with pytest.raises(ValueError, match=match):
        check_lists(ustart, ulen, ucols, NT, True, masks)


@pytest.mark.parametrize("kind", ["pair_out_of_range", "pair_twice", "order_out_of_range", "order_twice"])
def test_corrupt_launch_maps_raise(lists, kind):
    pairmap, order = lists["pairmap"].copy(), lists["order"].copy()
    if kind == "pair_out_of_range":
        pairmap[NT + 3] = NT
        match = "outside"
    elif kind == "pair_twice":
        pairmap[5] = pairmap[4]
        match = "twice"
    elif kind == "order_out_of_range":
        order[7] = order.size
        match = "outside"
    else:
        order[7] = order[8]
        match = "twice"
    with pytest.raises(ValueError, match=match):
        check_maps(pairmap, HEADS, NT, order)


def _quad_lists(L, masks):
    """Quad unions (entry = tile << 5 | partial << 4 | four member bits) of
    the four tiles each group of four pairmap slots names."""
    full = np.uint64(0xFFFFFFFFFFFFFFFF)
    ents = []
    for h in range(HEADS):
        for q in range(NT // 4):
            want = {}
            for k in range(4):
                r = h * NT + int(L["pairmap"][h * NT + 4 * q + k])
                for t in L["cols"][L["start"][r]: L["start"][r] + L["length"][r]]:
                    want[int(t)] = want.get(int(t), 0) | (1 << k)
            ents.append([t << 5 | (16 if masks is not None and masks[t] != full else 0) | b
                         for t, b in sorted(want.items())])
    qs = np.cumsum([0] + [len(e) for e in ents])[:-1]
    return qs, np.array([len(e) for e in ents], np.int32), np.array(sum(ents, []), np.int32)


@pytest.mark.parametrize("kind", ["valid", "valid_no_masks", "no_member_flag", "partial_flag_missing",
                                  "partial_flag_spurious", "tile_out_of_range"])
def test_quad_unions(lists, kind):
    L = lists
    masks = None if kind == "valid_no_masks" else L["masks"]
    qs, ql, qc = _quad_lists(L, masks)
    if kind.startswith("valid"):
        check_lists(qs, ql, qc, NT, 2, masks)
        return
    last = NT - 1
    hit = next(i for i in range(qc.size) if qc[i] >> 5 == last)
    other = next(i for i in range(qc.size) if qc[i] >> 5 != last)
    if kind == "no_member_flag":
        qc[other] &= ~15
        match = "belongs to no tile of its quad"
    elif kind == "partial_flag_missing":
        qc[hit] &= ~16
        match = "flagged full but its key mask is partial"
    elif kind == "partial_flag_spurious":
        qc[other] |= 16
        match = "flagged partial but its key mask is full"
    else:
        qc[hit] = (NT << 5) | 1
        match = "outside \\[0"
    with pytest.raises(ValueError, match=match):
        check_lists(qs, ql, qc, NT, 2, masks)
