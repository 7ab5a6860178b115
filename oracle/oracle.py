"""CPU parity oracle for the dynamic block-sparse attention path.

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg import this module, and only as the checker.
The product package ``prism_amd`` never imports it.

Two halves:
  * ``liboracle.so`` (bsa_oracle.c): the integer / canonical-fp32 selection
    path (zone statistics, shapes, geometry, pooling, scores, selection, list
    expansion and transpose), bit-exact targets for the HIP kernels;
  * numpy float64 attention forward/backward over per-tile key lists
    (``attn_fwd`` / ``attn_bwd``), the tolerance target for the MFMA kernels.

Reference functions followed are cited per wrapper (paths relative to
hymm/models/modules/ in the reference tree).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

ZONE_SIZE = 8
TILE = 64
CANDIDATES = [
    (4, 4, 4), (8, 2, 4), (8, 4, 2), (2, 4, 8), (2, 8, 4), (4, 2, 8), (4, 8, 2),
    (2, 8, 8), (8, 2, 8), (8, 8, 2), (4, 4, 8), (4, 8, 4), (8, 4, 4),
]


def build() -> str:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return os.path.join(_HERE, "liboracle.so")


def lib():
    global _LIB
    if _LIB is None:
        # PRISM_ORACLE_LIB: another build of the same source (the sanitizer
        # variant of the Makefile)
        path = os.environ.get("PRISM_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        _LIB = ctypes.CDLL(path)
        L = _LIB
        L.canon_exp.restype = ctypes.c_float
        L.canon_exp.argtypes = [ctypes.c_float]
        L.canon_log2.restype = ctypes.c_float
        L.canon_log2.argtypes = [ctypes.c_float]
        L.oc_cdf_threshold.restype = ctypes.c_uint64
        L.oc_cdf_threshold.argtypes = [ctypes.c_float]
        L.oc_tile_maps.restype = ctypes.c_int64
        L.oc_sum_lanes64.restype = ctypes.c_float
        L.oc_local_of_rearr.restype = ctypes.c_int
    return _LIB


def _p(a: Optional[np.ndarray]):
    # data_as keeps a reference to the array, so a temporary made inside an
    # argument list (np.ascontiguousarray copy) lives until the call returns
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _dtype_code(a: np.ndarray) -> int:
    if a.dtype == np.float32:
        return 0
    if a.dtype == np.uint16:  # bf16 bit patterns
        return 1
    raise TypeError(f"unsupported dtype {a.dtype}")


# ---------------------------------------------------------------- bf16 helpers
def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- scalar math
def canon_exp(x: float) -> float:
    return lib().canon_exp(ctypes.c_float(x))


def canon_log2(x: float) -> float:
    return lib().canon_log2(ctypes.c_float(x))


def cdf_threshold(p: float) -> int:
    return int(lib().oc_cdf_threshold(ctypes.c_float(p)))


def sum_lanes64(vals: np.ndarray) -> float:
    v = np.ascontiguousarray(vals, dtype=np.float32)
    return lib().oc_sum_lanes64(_p(v), ctypes.c_int(v.size))


# ---------------------------------------------------------------- zone stats
def zone_stats(v: np.ndarray, grid, valid: Optional[np.ndarray] = None):
    """compute_zone_aggregates on v[0].mean(0) (dynamic_block_shape.py:68-129,
    dynamic_block_attention.py:236).  v: [B,H,S,D] float32 or bf16 bits."""
    T, Hg, Wg = grid
    B, H, S, D = v.shape
    v = np.ascontiguousarray(v)
    Nz = (T // 8) * (Hg // 8) * (Wg // 8)
    packed = np.zeros((Nz, 25 * D), np.float32)
    av = np.zeros((Nz, 24), np.uint8)
    vm = None if valid is None else np.ascontiguousarray(valid, dtype=np.uint8)
    lib().oc_zone_stats(_p(v), _dtype_code(v), H, ctypes.c_int64(S), D, _p(vm), T, Hg, Wg, _p(packed), _p(av))
    return packed, av


def zone_gradient(packed: np.ndarray, axis_valid: np.ndarray, D: int):
    """Per-zone rho_raw and anisotropy (dynamic_block_shape.py:248-289)."""
    Nz = packed.shape[0]
    rho_raw = np.zeros(Nz, np.float32)
    aniso = np.zeros((Nz, 3), np.float32)
    lib().oc_zone_gradient(_p(np.ascontiguousarray(packed)), _p(np.ascontiguousarray(axis_valid)), Nz, D,
                           _p(rho_raw), _p(aniso))
    return rho_raw, aniso


def audio_zone_stats(norms: np.ndarray, grid, valid: Optional[np.ndarray] = None):
    """Per-zone audio mean and directional variances
    (dynamic_block_shape.py:189-245, before max-normalisation)."""
    T, Hg, Wg = grid
    Nz = (T // 8) * (Hg // 8) * (Wg // 8)
    n = np.ascontiguousarray(norms)
    abar = np.zeros(Nz, np.float32)
    vhat = np.zeros((Nz, 3), np.float32)
    vm = None if valid is None else np.ascontiguousarray(valid, dtype=np.uint8)
    lib().oc_audio_zone_stats(_p(n), _dtype_code(n), _p(vm), T, Hg, Wg, _p(abar), _p(vhat))
    return abar, vhat


def zone_shapes(rho_raw, aniso, abar=None, vhat=None, method="ivpq", lambda_a=0.5,
                tau_128=0.15, lambda_128=1.0):
    """select_shapes_ivpq / select_shapes_penalty (dynamic_block_shape.py:303-355)."""
    if method not in ("ivpq", "penalty"):
        raise ValueError(f"unknown dynamic-block method: {method!r}")
    Nz = rho_raw.shape[0]
    g = np.zeros((Nz, 3), np.float32)
    rho = np.zeros(Nz, np.float32)
    sid = np.zeros(Nz, np.int64)
    ab = None if abar is None else np.ascontiguousarray(abar, dtype=np.float32)
    vh = None if vhat is None else np.ascontiguousarray(vhat, dtype=np.float32)
    lib().oc_zone_shapes(_p(np.ascontiguousarray(rho_raw, dtype=np.float32)),
                         _p(np.ascontiguousarray(aniso, dtype=np.float32)), _p(ab), _p(vh), Nz,
                         0 if method == "ivpq" else 1, ctypes.c_float(lambda_a), ctypes.c_float(tau_128),
                         ctypes.c_float(lambda_128), _p(g), _p(rho), _p(sid))
    return g, rho, sid


def select_zone_shapes(v, audio_norms, grid, method, lambda_a=0.5, tau_128=0.15, lambda_128=1.0,
                       valid=None):
    """End-to-end select_zone_shapes (dynamic_block_shape.py:358-391)."""
    D = v.shape[-1]
    packed, av = zone_stats(v, grid, valid)
    rho_raw, aniso = zone_gradient(packed, av, D)
    abar = vhat = None
    if audio_norms is not None:
        abar, vhat = audio_zone_stats(audio_norms, grid, valid)
    return zone_shapes(rho_raw, aniso, abar, vhat, method, lambda_a, tau_128, lambda_128)[2]


def a2v_norms(res: np.ndarray, out_bf16: bool):
    """residual[0].norm(dim=-1) (wan_video_dit.py:742-752).  res: [S, C]."""
    r = np.ascontiguousarray(res)
    S, C = r.shape
    out = np.zeros(S, np.uint16 if out_bf16 else np.float32)
    lib().oc_a2v_norms(_p(r), _dtype_code(r), ctypes.c_int64(S), C, _p(out), 1 if out_bf16 else 0)
    return out


# ---------------------------------------------------------------- geometry
def rearrange_index(shape_ids: np.ndarray, grid):
    """_build_rearrange_index (dynamic_block_attention.py:107-135)."""
    T, Hg, Wg = grid
    S = T * Hg * Wg
    sid = np.ascontiguousarray(shape_ids, dtype=np.int64)
    src = np.zeros(S, np.int64)
    inv = np.zeros(S, np.int64)
    lib().oc_rearrange_index(_p(sid), T, Hg, Wg, _p(src), _p(inv))
    return src, inv


def tile_maps(shape_ids: np.ndarray):
    """_build_block_tile_maps (dynamic_block_attention.py:138-170)."""
    sid = np.ascontiguousarray(shape_ids, dtype=np.int64)
    Nz = sid.shape[0]
    bot = np.zeros(Nz * 8, np.int64)
    boff = np.zeros(Nz, np.int64)
    nb = int(lib().oc_tile_maps(_p(sid), Nz, _p(bot), None, _p(boff)))
    kbt = np.zeros((nb + 1, 2), np.int64)
    lib().oc_tile_maps(_p(sid), Nz, _p(bot), _p(kbt), _p(boff))
    return bot, kbt, nb, boff


def block_pool(x: np.ndarray, shape_ids, grid, valid=None):
    """Masked logical-block means, fp32 (bsa_interface.py:177-201,
    dynamic_block_attention.py:173-188).  x: [B,H,S,D] THW (padded)."""
    T, Hg, Wg = grid
    B, H, S, D = x.shape
    sid = np.ascontiguousarray(shape_ids, dtype=np.int64)
    _, _, nb, _ = tile_maps(sid)
    out = np.zeros((B, H, nb, D), np.float32)
    bc = np.zeros(nb, np.int32)
    tc = np.zeros(S // TILE, np.int32)
    vm = None if valid is None else np.ascontiguousarray(valid, dtype=np.uint8)
    xx = np.ascontiguousarray(x)
    lib().oc_block_pool(_p(xx), _dtype_code(xx), B, H, ctypes.c_int64(S), D, _p(vm), _p(sid), T, Hg, Wg,
                        _p(out), _p(bc), _p(tc))
    return out, bc, tc


# ---------------------------------------------------------------- uniform chunk layout
def padded_grid(grid, chunk):
    """Grid rounded up to multiples of the chunk (bsa_interface.py:1318-1331)."""
    return tuple(-(-g // c) * c for g, c in zip(grid, chunk))


def chunk_source_index(grid, pgrid, chunk, rows: Optional[int] = None) -> np.ndarray:
    """rearrange_THW_to_3d_block (bsa_interface.py:1105-1109) as a source
    index over the padded grid: src[p] = THW token (of the unpadded grid) of
    rearranged row p, -1 for padding (tokens outside the grid, and rows
    p >= Tp*Hp*Wp up to ``rows``)."""
    T, H, W = grid
    Tp, Hp, Wp = pgrid
    ct, ch, cw = chunk
    t = np.arange(Tp)[:, None, None]
    h = np.arange(Hp)[None, :, None]
    w = np.arange(Wp)[None, None, :]
    tok = np.where((t < T) & (h < H) & (w < W), (t * H + h) * W + w, -1)
    src = tok.reshape(Tp // ct, ct, Hp // ch, ch, Wp // cw, cw).transpose(0, 2, 4, 1, 3, 5).reshape(-1)
    if rows is not None and rows > src.size:
        src = np.concatenate([src, np.full(rows - src.size, -1, src.dtype)])
    return src.astype(np.int64)


def chunk_pool(x: np.ndarray, src: np.ndarray, valid: Optional[np.ndarray], csz: int, n_blocks: int):
    """(masked_)mean_pooling_compression (bsa_interface.py:164-201) of the
    rearranged rows: per chunk, its valid rows j fall into RPI = 512 / D row
    groups (j mod RPI), each summed in fp32 in row order from +0; the chunk
    sum is ((p_0 + p_1) + ...) + p_{RPI-1}, divided by max(count, 1).
    x: [B,H,S_in,D] float32 (bf16 values widened).  Returns (means
    [B,H,n_blocks,D] fp32, counts [n_blocks])."""
    x = np.asarray(x, np.float32)
    rows = src[: n_blocks * csz].reshape(n_blocks, csz)
    ok = rows >= 0
    if valid is not None:
        ok &= np.asarray(valid).astype(bool)[np.maximum(rows, 0)]
    B, H, _, D = x.shape
    rpi = 512 // D
    part = np.zeros((rpi, B, H, n_blocks, D), np.float32)
    for j in range(csz):
        xj = x[:, :, np.maximum(rows[:, j], 0), :]
        part[j % rpi] = np.where(ok[None, None, :, j, None], part[j % rpi] + xj, part[j % rpi])
    acc = part[0]
    for r in range(1, rpi):
        acc = (acc + part[r]).astype(np.float32)
    cnt = ok.sum(axis=1).astype(np.int32)
    mean = acc / np.maximum(cnt, 1).astype(np.float32)[None, None, :, None]
    return mean.astype(np.float32), cnt


def chunk_rows(x: np.ndarray, src: np.ndarray) -> np.ndarray:
    """Rearranged rows [B,H,len(src),D] with zero rows at padding."""
    out = np.zeros(x.shape[:2] + (src.size, x.shape[3]), x.dtype)
    ok = src >= 0
    out[:, :, ok] = x[:, :, src[ok]]
    return out


def chunk_kblock_tiles(n_blocks: int, csz: int, Nt: int) -> np.ndarray:
    """[n_blocks + 1, 2] tiles of each chunk (second = Nt for 64-token chunks),
    the kblock_tiles form expand_tiles takes."""
    b = np.arange(n_blocks + 1, dtype=np.int64)
    if csz == 64:
        kbt = np.stack([b, np.full_like(b, Nt)], 1)
    else:
        kbt = np.stack([2 * b, 2 * b + 1], 1)
    kbt[n_blocks] = Nt
    return kbt


def uniform_pipeline(q, k, q_grid, k_grid, chunk_q, chunk_k, *, sparsity=0.875, cdf_threshold_p=None,
                     q_valid=None, k_valid=None, q_pad_rows=None, k_pad_rows=None, skip_padded_queries=False):
    """Selection half of _attention_bsa.forward (bsa_interface.py:600-640) on
    the uniform chunk layout: rearranged rows, pooled means, fp32 scores (no
    invalid-key fill), selection, per-query-tile key-tile lists.  q/k:
    [B,H,S,D] THW float32; q_valid/k_valid: THW validity or None (padding of
    the grid is always invalid); *_pad_rows: rows per head (multiple of 128)."""
    B, H, _, D = q.shape
    sm_scale = 1.0 / (D ** 0.5)
    side = {}
    for name, x, grid, chunk, valid, rows in (("q", q, q_grid, chunk_q, q_valid, q_pad_rows),
                                               ("k", k, k_grid, chunk_k, k_valid, k_pad_rows)):
        pg = padded_grid(grid, chunk)
        csz = int(np.prod(chunk))
        Sp = int(np.prod(pg))
        rows = rows or -(-Sp // 128) * 128
        src = chunk_source_index(grid, pg, chunk, rows)
        nb = Sp // csz
        mean, cnt = chunk_pool(x, src, valid, csz, nb)
        okrow = src >= 0
        if valid is not None:
            okrow &= np.asarray(valid).astype(bool)[np.maximum(src, 0)]
        side[name] = dict(pgrid=pg, csz=csz, src=src, nb=nb, mean=mean, count=cnt, rows=rows, Nt=rows // TILE,
                          valid_re=okrow.astype(np.uint8),
                          tile_count=okrow.reshape(-1, TILE).sum(1).astype(np.int32),
                          masked=valid is not None or bool((src[:Sp] < 0).any()) or rows > Sp)
    sq, sk = side["q"], side["k"]
    scores = block_scores(sq["mean"].reshape(B * H, sq["nb"], D), sk["mean"].reshape(B * H, sk["nb"], D), None)
    sel, nsel = select(scores, sparsity, cdf_threshold_p, sm_scale)
    kbt = chunk_kblock_tiles(sk["nb"], sk["csz"], sk["Nt"])
    tiles, ntiles = expand_tiles(sel, nsel, kbt, sk["Nt"], sk["tile_count"] if sk["masked"] else None)
    tcap = tiles.shape[1]
    tpb_q = sq["csz"] // TILE
    Ntq = sq["Nt"]
    bid = np.minimum(np.arange(Ntq) // tpb_q, sq["nb"] - 1)
    rows_q = (np.arange(B * H)[:, None] * sq["nb"] + bid[None, :]).reshape(-1)
    qstart = rows_q * tcap
    qlen = ntiles[rows_q].astype(np.int32)
    empty_q = sq["tile_count"] == 0
    pad_tiles = np.arange(Ntq) * TILE >= int(np.prod(sq["pgrid"]))
    drop = pad_tiles | (empty_q if (skip_padded_queries and sq["masked"]) else np.zeros(Ntq, bool))
    qlen = np.where(np.tile(drop, B * H), 0, qlen).astype(np.int32)
    return dict(q=sq, k=sk, scores=scores, sel=sel, nsel=nsel, tiles=tiles, ntiles=ntiles, qstart=qstart, qlen=qlen,
                qcols=tiles.reshape(-1))


def block_scores(qc: np.ndarray, kc: np.ndarray, block_count: Optional[np.ndarray]):
    """cal_score + invalid-key fill (bsa_interface.py:203-207,
    dynamic_block_attention.py:276-279).  qc: [BH, Nq, D], kc: [BH, Nk, D]
    fp32 -> [BH, Nq, Nk]."""
    BH, Nq, D = qc.shape
    Nk = kc.shape[1]
    out = np.zeros((BH, Nq, Nk), np.float32)
    bc = None if block_count is None else np.ascontiguousarray(block_count, dtype=np.int32)
    lib().oc_block_scores(_p(np.ascontiguousarray(qc, dtype=np.float32)),
                          _p(np.ascontiguousarray(kc, dtype=np.float32)), _p(bc), BH, ctypes.c_int64(Nq),
                          ctypes.c_int64(Nk), D, _p(out))
    return out


def selection_params(N: int, sparsity: Optional[float], cdf_threshold_p: Optional[float]):
    """(mode, k_lo, ub) exactly as bsa_interface.py:235-304 derives them."""
    if sparsity is not None and cdf_threshold_p is None:
        k = int((1 - sparsity) * N)
        return 0, k, k
    if sparsity is None and cdf_threshold_p is not None:
        ub = min(N, int(cdf_threshold_p * N) + 1)
        return 1, 1, ub
    if sparsity is not None and cdf_threshold_p is not None:
        kt = max(1, int((1 - sparsity) * N))
        ub = min(N, max(kt, int(cdf_threshold_p * N) + 1))
        return 2, kt, ub
    raise ValueError("Either sparsity or cdf_threshold must be provided")


def select(scores: np.ndarray, sparsity, cdf_threshold_p, sm_scale: float):
    """Per-row block selection; returns (sel [rows, cap] int64, nsel [rows])."""
    rows = int(np.prod(scores.shape[:-1]))
    N = scores.shape[-1]
    mode, k_lo, ub = selection_params(N, sparsity, cdf_threshold_p)
    cap = max(ub, 1)
    sel = np.full((rows, cap), -1, np.int64)
    nsel = np.zeros(rows, np.int32)
    thr = cdf_threshold(cdf_threshold_p) if mode != 0 else 0
    lib().oc_select(_p(np.ascontiguousarray(scores, dtype=np.float32)), ctypes.c_int64(rows), ctypes.c_int64(N),
                    mode, ctypes.c_int64(k_lo), ctypes.c_int64(ub), ctypes.c_float(sm_scale), ctypes.c_uint64(thr),
                    ctypes.c_int64(cap), _p(sel), _p(nsel))
    return sel, nsel


def expand_tiles(sel, nsel, kblock_tiles, Nt, tile_count=None):
    """Selected blocks -> tile lists (dynamic_block_attention.py:297-319)."""
    rows, cap = sel.shape
    tcap = 2 * cap
    tiles = np.full((rows, tcap), -1, np.int32)
    nt = np.zeros(rows, np.int32)
    tc = None if tile_count is None else np.ascontiguousarray(tile_count, dtype=np.int32)
    lib().oc_expand_tiles(_p(np.ascontiguousarray(sel)), _p(np.ascontiguousarray(nsel)), ctypes.c_int64(rows),
                          ctypes.c_int64(cap), _p(np.ascontiguousarray(kblock_tiles, dtype=np.int64)),
                          ctypes.c_int64(Nt), _p(tc), ctypes.c_int64(tcap), _p(tiles), _p(nt))
    return tiles, nt


def transpose_lists(qstart, qlen, qcols, BH, Nt, Ntk=None):
    """k-tile -> ascending q-tile lists (bsa_interface.py:147-161).  Nt query
    tiles per head listing key tiles < Ntk (default Nt)."""
    Ntk = Nt if Ntk is None else Ntk
    kcols = np.full(BH * Ntk * Nt, -1, np.int32)
    klen = np.zeros(BH * Ntk, np.int32)
    lib().oc_transpose_lists(_p(np.ascontiguousarray(qstart, dtype=np.int64)),
                             _p(np.ascontiguousarray(qlen, dtype=np.int32)),
                             _p(np.ascontiguousarray(qcols, dtype=np.int32)), BH, ctypes.c_int64(Nt),
                             ctypes.c_int64(Ntk), _p(kcols), _p(klen))
    return kcols.reshape(BH * Ntk, Nt), klen


def tile_masks(valid: np.ndarray) -> np.ndarray:
    """Key validity per 64-token tile as a 64-bit word, bit j = token j valid
    (the kv_valid_mask of bsa_interface.py:328-385 regrouped per tile)."""
    v = (np.asarray(valid).reshape(-1, TILE) != 0).astype(np.uint64)
    return (v << np.arange(TILE, dtype=np.uint64)[None, :]).sum(axis=1, dtype=np.uint64)


def _matching(m: int, g: int):
    """Matching m of g rows: the first free row pairs with the
    (m mod (free - 1))-th other free row, then m //= free - 1, and so on."""
    free = list(range(g))
    pairs = []
    while free:
        a = free[0]
        c = m % (len(free) - 1)
        m //= len(free) - 1
        b = free[1 + c]
        pairs.append((a, b))
        free = [x for x in free[1:] if x != b]
    return pairs


def pair_tiles(start, length, cols, Nt, col_tiles=None, group=8):
    """Pairing of the tiles of each group of `group` consecutive tiles of a
    head that maximises the summed list overlap of its pairs (ties: the lowest
    matching index of _matching).  Returns pairmap [rows] int32 (indices
    inside the head); pair p of a head is (pairmap[2p], pairmap[2p+1]).  No
    reference counterpart: it only chooses which tiles share a workgroup."""
    start = np.asarray(start, np.int64)
    length = np.asarray(length, np.int64)
    cols = np.asarray(cols, np.int64)
    col_tiles = Nt if col_tiles is None else col_tiles
    rows = start.size
    out = np.zeros(rows, np.int32)
    for h in range(rows // Nt):
        for r0 in range(0, Nt, group):
            g = min(group, Nt - r0)
            sets = []
            for i in range(g):
                r = h * Nt + r0 + i
                li = cols[start[r]: start[r] + length[r]]
                sets.append(set(int(x) for x in li if 0 <= x < col_tiles))
            nm = 1
            for f in range(g - 1, 0, -2):
                nm *= f
            best = None
            for m in range(nm):
                pairs = _matching(m, g)
                total = sum(len(sets[a] & sets[b]) for a, b in pairs)
                if best is None or total > best[0]:
                    best = (total, pairs)
            for k, (a, b) in enumerate(best[1]):
                out[h * Nt + r0 + 2 * k] = r0 + a
                out[h * Nt + r0 + 2 * k + 1] = r0 + b
    return out


def pair_union(start, length, cols, Nt, masks=None, pairmap=None):
    """For each row pair (2p, 2p+1), or the rows pairmap pairs inside each
    head of Nt rows: the ascending union of the two rows' tile lists,
    entry = tile << 3 | partial << 2 | in_second << 1 | in_first,
    partial = masks is given and masks[tile] is not all ones.  This is the
    work list of the paired-tile attention kernels (no reference counterpart:
    the reference walks one list per tile, bsa_interface.py:328-523)."""
    start = np.asarray(start, np.int64)
    length = np.asarray(length, np.int64)
    cols = np.asarray(cols, np.int64)
    out = []
    for p in range(start.size // 2):
        if pairmap is None:
            ra, rb = 2 * p, 2 * p + 1
        else:
            h0 = (2 * p) // Nt * Nt
            ra, rb = h0 + int(pairmap[2 * p]), h0 + int(pairmap[2 * p + 1])
        a = cols[start[ra]: start[ra] + length[ra]]
        b = cols[start[rb]: start[rb] + length[rb]]
        u = np.union1d(a, b)
        e = (u << 3) | np.isin(u, a).astype(np.int64) | (np.isin(u, b).astype(np.int64) << 1)
        if masks is not None:
            e |= (np.asarray(masks, np.uint64)[u] != np.uint64(0xFFFFFFFFFFFFFFFF)).astype(np.int64) << 2
        out.append(e.astype(np.int32))
    return out


# ---------------------------------------------------------------- full selection pipeline
def select_pipeline(q, k, v, grid, *, method="ivpq", sparsity=0.9375, cdf_threshold_p=None,
                    audio_norms=None, valid=None, lambda_a=0.5, tau_128=0.15, lambda_128=1.0,
                    shape_ids=None, skip_padded_queries=False):
    """Steps (1)-(5) of flash_attn_bsa_3d_dynamic
    (dynamic_block_attention.py:233-319): shape ids, geometry, pooled block
    means, scores, selection, per-q-tile key-tile lists.  Inputs are THW
    [B,H,S,D] float32 or bf16 bit arrays."""
    B, H, S, D = q.shape
    T, Hg, Wg = grid
    sm_scale = 1.0 / (D ** 0.5)
    if shape_ids is None:
        shape_ids = select_zone_shapes(v, audio_norms, grid, method, lambda_a, tau_128, lambda_128, valid)
    bot, kbt, nb, boff = tile_maps(shape_ids)
    Nt = S // TILE
    qc, bc, tc = block_pool(q, shape_ids, grid, valid)
    kc, _, _ = block_pool(k, shape_ids, grid, valid)
    scores = block_scores(qc.reshape(B * H, nb, D), kc.reshape(B * H, nb, D), bc if valid is not None else None)
    sel, nsel = select(scores, sparsity, cdf_threshold_p, sm_scale)
    tiles, ntiles = expand_tiles(sel, nsel, kbt, Nt, tc if valid is not None else None)
    tcap = tiles.shape[1]
    # per q tile: the row of its block
    rows = (np.arange(B * H)[:, None] * nb + bot[None, :]).reshape(-1)
    qstart = rows * tcap
    qlen = ntiles[rows]
    if skip_padded_queries and valid is not None:
        # query tiles without a valid token attend to nothing
        qlen = np.where(np.tile(tc == 0, B * H), 0, qlen).astype(np.int32)
    return dict(shape_ids=shape_ids, block_id_of_tile=bot, kblock_tiles=kbt, N_b=nb, block_offset=boff,
                q_cmp=qc, k_cmp=kc, block_count=bc, tile_count=tc, scores=scores, sel=sel, nsel=nsel,
                tiles=tiles, ntiles=ntiles, qstart=qstart, qlen=qlen, qcols=tiles.reshape(-1))


# ---------------------------------------------------------------- attention (float64)
def _row_keys(qcols, start, n):
    cols = qcols[start:start + n].astype(np.int64)
    return (cols[:, None] * TILE + np.arange(TILE)[None, :]).reshape(-1)


def attn_fwd(q, k, v, qstart, qlen, qcols, kv_valid, sm_scale):
    """Block-sparse attention forward over per-tile key lists
    (flash_attn_bsa_varlen_mask.py:191-319).  q,k,v: [BH, S, D] tile order.
    Returns o [BH,S,D] float64 and natural-log lse [BH,S] (-inf for rows
    with no valid key, whose output is 0)."""
    BH, S, D = q.shape
    Nt = S // TILE
    q = q.astype(np.float64); k = k.astype(np.float64); v = v.astype(np.float64)
    o = np.zeros((BH, S, D)); lse = np.full((BH, S), -np.inf)
    for bh in range(BH):
        for t in range(Nt):
            row = bh * Nt + t
            n = int(qlen[row])
            if n == 0:
                continue
            idx = _row_keys(qcols, int(qstart[row]), n)
            s = q[bh, t * TILE:(t + 1) * TILE] @ k[bh, idx].T * sm_scale
            if kv_valid is not None:
                s[:, ~kv_valid[idx].astype(bool)] = -np.inf
            m = s.max(axis=1)
            ok = np.isfinite(m)
            if not ok.any():
                continue
            p = np.zeros_like(s)
            p[ok] = np.exp(s[ok] - m[ok, None])
            l = p.sum(axis=1)
            ot = np.zeros((TILE, D))
            ot[ok] = (p[ok] @ v[bh, idx]) / l[ok, None]
            o[bh, t * TILE:(t + 1) * TILE] = ot
            lt = np.full(TILE, -np.inf)
            lt[ok] = m[ok] + np.log(l[ok])
            lse[bh, t * TILE:(t + 1) * TILE] = lt
    return o, lse


def _round_bf16(x: np.ndarray) -> np.ndarray:
    """float64 -> nearest bf16 value (via float32, ties to even), as float64."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x.astype(np.float32))).astype(np.float64)


def attn_bwd_term_magnitudes(q, k, v, o, do, lse, qstart, qlen, qcols, kv_valid, sm_scale):
    """Per element of dQ, dK, dV the sum of the magnitudes of the terms that
    attn_bwd adds up: sum_k |dS_qk| |K_k| sm_scale, sum_q |dS_qk| |Q_q|
    sm_scale and sum_q P_qk |dO_q| (float64, same lists and masks).  Rounding
    each dS (P) operand to bf16 moves an element by at most 2^-9 times this
    sum, the bound of the reference kernels' own arithmetic against float64."""
    BH, S, D = q.shape
    Nt = S // TILE
    q = q.astype(np.float64); k = k.astype(np.float64); v = v.astype(np.float64)
    o = o.astype(np.float64); do = do.astype(np.float64)
    delta = (o * do).sum(-1)
    mq = np.zeros_like(q); mk = np.zeros_like(k); mv = np.zeros_like(v)
    for bh in range(BH):
        for t in range(Nt):
            row = bh * Nt + t
            n = int(qlen[row])
            if n == 0:
                continue
            sl = slice(t * TILE, (t + 1) * TILE)
            idx = _row_keys(qcols, int(qstart[row]), n)
            s = q[bh, sl] @ k[bh, idx].T * sm_scale
            if kv_valid is not None:
                s[:, ~kv_valid[idx].astype(bool)] = -np.inf
            L = lse[bh, sl]
            p = np.zeros_like(s)
            ok = np.isfinite(L)
            p[ok] = np.exp(s[ok] - L[ok, None])
            ds = np.abs(p * (do[bh, sl] @ v[bh, idx].T - delta[bh, sl][:, None]))
            mq[bh, sl] += ds @ np.abs(k[bh, idx]) * sm_scale
            mk[bh, idx] += ds.T @ np.abs(q[bh, sl]) * sm_scale
            mv[bh, idx] += p.T @ np.abs(do[bh, sl])
    return mq, mk, mv


def attn_bwd(q, k, v, o, do, lse, qstart, qlen, qcols, kv_valid, sm_scale, bf16_operands=False):
    """Backward of attn_fwd (bsa_interface.py:387-523 semantics: delta =
    rowsum(o * do), dK and dQ scaled by sm_scale).  float64.

    bf16_operands: round the two computed matrix operands to bf16 before
    their products, as the reference's kernels do: P (from the final LSE) for
    dV = P^T dO (flash_attn_bsa_varlen_mask.py:382-391), dS = P (dP - delta),
    formed from the unrounded P, for dK = dS^T Q and dQ = dS K (:395-399,
    :462-470).  Everything else stays float64.  Where dK / dQ sum terms of
    mixed sign to a small result, this rounding alone moves them by up to
    2^-9 of the sum of the terms' magnitudes, more than the result's own bf16
    rounding."""
    rb = _round_bf16 if bf16_operands else (lambda x: x)
    BH, S, D = q.shape
    Nt = S // TILE
    q = q.astype(np.float64); k = k.astype(np.float64); v = v.astype(np.float64)
    o = o.astype(np.float64); do = do.astype(np.float64)
    delta = (o * do).sum(-1)
    dq = np.zeros_like(q); dk = np.zeros_like(k); dv = np.zeros_like(v)
    for bh in range(BH):
        for t in range(Nt):
            row = bh * Nt + t
            n = int(qlen[row])
            if n == 0:
                continue
            sl = slice(t * TILE, (t + 1) * TILE)
            idx = _row_keys(qcols, int(qstart[row]), n)
            s = q[bh, sl] @ k[bh, idx].T * sm_scale
            if kv_valid is not None:
                s[:, ~kv_valid[idx].astype(bool)] = -np.inf
            L = lse[bh, sl]
            p = np.zeros_like(s)
            ok = np.isfinite(L)
            p[ok] = np.exp(s[ok] - L[ok, None])
            dv[bh, idx] += rb(p).T @ do[bh, sl]
            dp = do[bh, sl] @ v[bh, idx].T
            ds = p * (dp - delta[bh, sl][:, None])
            dq[bh, sl] += rb(ds) @ k[bh, idx] * sm_scale
            dk[bh, idx] += rb(ds).T @ q[bh, sl] * sm_scale
    return dq, dk, dv
