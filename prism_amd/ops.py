"""Tensor-level wrappers over the prism_bsa kernels.

Every computation runs in libprism_bsa.so, reached through its PyTorch
operator registration (torch.ops.prism.*, libprism_torch.so): each operator
allocates its outputs through the caching allocator and launches on the
current HIP stream.  Inputs must be GPU tensors; they are made contiguous
where the kernels need it.
"""
from __future__ import annotations

import contextlib
import os
from typing import Dict, List, Optional, Tuple

import torch

from . import _lib  # noqa: F401  (the ctypes binding of the same C-ABI, for C-ABI-level callers and tests)
from . import _torch_ops

F32, BF16 = 0, 1
_ops = _torch_ops.load()
_CANDIDATES = 13  # entries of the candidate shape table (dynamic_block_shape.py:6-27)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


# Optional per-entry-point timing: when enabled, every C-ABI call is bracketed
# by a pair of HIP events on the stream it is launched on (the current stream).
_timings: Optional[Dict[str, List[Tuple[torch.cuda.Event, torch.cuda.Event]]]] = None


@contextlib.contextmanager
def kernel_timing():
    """Record HIP events around every C-ABI launch made inside the block.
    Yields a dict name -> list of (start, end) events; after a synchronize,
    ``summarize(d)`` gives per-entry-point call counts and average ms."""
    global _timings
    prev, _timings = _timings, {}
    try:
        yield _timings
    finally:
        _timings = prev


def summarize(timings) -> Dict[str, Tuple[int, float]]:
    return {name: (len(ev), sum(a.elapsed_time(b) for a, b in ev) / len(ev)) for name, ev in timings.items() if ev}


def _op(name: str, *args):
    """torch.ops.prism.<name>(*args), timed under kernel_timing() (key
    "prism_<name>", the C-ABI entry point the operator wraps; launches on the
    side stream get the key "prism_<name> (side stream)": their time includes
    waiting there for CUs that the main stream's kernels hold)."""
    fn = getattr(_ops, name)
    if _timings is None:
        return fn(*args)
    cur = torch.cuda.current_stream()
    key = "prism_" + name + (" (side stream)" if any(cur == s for s in _side_streams.values()) else "")
    st = torch.cuda.Event(enable_timing=True)
    en = torch.cuda.Event(enable_timing=True)
    st.record()
    out = fn(*args)
    en.record()
    _timings.setdefault(key, []).append((st, en))
    return out


def _opt(t: torch.Tensor) -> Optional[torch.Tensor]:
    """Empty placeholder outputs of the operators -> None."""
    return None if t.numel() == 0 and t.dim() == 1 and t.dtype == torch.float32 else t


def _code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.bfloat16:
        return BF16
    raise TypeError(f"prism_amd: unsupported dtype {t.dtype} (float32 or bfloat16)")


def _cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("prism_amd: tensors must live on the GPU (no CPU path)")


def _grid(grid) -> Tuple[int, int, int]:
    T, H, W = (int(x) for x in grid)
    return T, H, W


def _u8(valid: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    if valid is None:
        return None
    return valid.contiguous().view(torch.uint8) if valid.dtype == torch.bool else valid.contiguous().to(torch.uint8)


# ------------------------------------------------------------------ statistics
def zone_stats(v: torch.Tensor, grid, valid: Optional[torch.Tensor] = None, box=None):
    """[B,H,S,D] THW -> packed [Nz, 25D] fp32, axis_valid [Nz, 24] uint8.
    grid is the zone grid (multiples of 8); box the input grid inside it that
    v and valid cover (default: the zone grid itself)."""
    _cuda(v, valid)
    v = v.contiguous()
    B, H, S, D = v.shape
    T, Hg, Wg = _grid(grid)
    Ti, Hi, Wi = _grid(box if box is not None else grid)
    _code(v)
    return _op("zone_stats", v, _u8(valid), [T, Hg, Wg], [Ti, Hi, Wi])


def audio_zone_stats(norms: torch.Tensor, grid, valid: Optional[torch.Tensor] = None, box=None):
    _cuda(norms, valid)
    norms = norms.contiguous()
    T, Hg, Wg = _grid(grid)
    Ti, Hi, Wi = _grid(box if box is not None else grid)
    _code(norms)
    return _op("audio_zone_stats", norms, _u8(valid), [T, Hg, Wg], [Ti, Hi, Wi])


def zone_gradient(packed: torch.Tensor, axis_valid: torch.Tensor, D: int):
    _cuda(packed, axis_valid)
    return _op("zone_gradient", packed, axis_valid, int(D))


def zone_shapes(rho_raw, aniso, abar, vhat, method: str, lambda_a: float, tau_128: float, lambda_128: float):
    if method not in ("ivpq", "penalty"):
        raise ValueError(f"unknown dynamic-block method: {method!r}")
    _cuda(rho_raw, aniso, abar, vhat)
    return _op("zone_shapes", rho_raw, aniso, abar, vhat, 0 if method == "ivpq" else 1, float(lambda_a),
               float(tau_128), float(lambda_128))


def assign_shapes(g: torch.Tensor, rho: torch.Tensor, method: int, tau_128: float, lambda_128: float) -> torch.Tensor:
    """select_shapes_ivpq (method 0) / select_shapes_penalty (method 1) on given g, rho."""
    _cuda(g, rho)
    return _op("assign_shapes", g.contiguous().float(), rho.contiguous().float(), int(method), float(tau_128),
               float(lambda_128))


def a2v_norms(residual: torch.Tensor) -> torch.Tensor:
    """Per-token L2 norm of batch 0: [B,S,C] (or [S,C]) -> [S] in the input dtype."""
    _cuda(residual)
    r = residual[0] if residual.dim() == 3 else residual
    _code(r)
    return _op("a2v_norms", r.contiguous())


def linear_rownorm(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
                   norms_dtype: Optional[torch.dtype] = None):
    """y = x weight^T + bias (bf16, fp32 accumulate) and the L2 norm of every
    row of the stored y, fused: [M, K] x [N, K] -> ([M, N], [M]).  N must be a
    multiple of 256 and K of 64."""
    _cuda(x, weight, bias)
    nd = x.dtype if norms_dtype is None else norms_dtype
    code = F32 if nd == torch.float32 else BF16 if nd == torch.bfloat16 else None
    if code is None:
        raise TypeError(f"prism_amd: unsupported dtype {nd} (float32 or bfloat16)")
    return _op("linear_rownorm", _bf16(x, "x"), _bf16(weight, "weight"), None if bias is None else _bf16(bias, "bias"),
               code)


# ------------------------------------------------------------------ geometry
class ZoneLayout:
    """Per-call block/tile bookkeeping for one set of shape ids.

    grid is the zone grid (multiples of 8); box is the input grid inside it
    (default: the zone grid).  THW tensors of this layout hold S_in =
    prod(box) tokens per head, tile-order tensors S = prod(grid) rows; grid
    positions outside the box are padding (zero, invalid)."""

    def __init__(self, shape_ids: torch.Tensor, grid, box=None):
        _cuda(shape_ids)
        self.grid = _grid(grid)
        self.box = _grid(box) if box is not None else self.grid
        T, Hg, Wg = self.grid
        if not all(0 < b <= g for b, g in zip(self.box, self.grid)):
            raise ValueError(f"input grid {self.box} must fit the zone grid {self.grid}")
        self.padded = self.box != self.grid
        self.Nz = (T // 8) * (Hg // 8) * (Wg // 8)
        self.Nt = self.Nz * 8
        self.S = T * Hg * Wg
        self.S_in = self.box[0] * self.box[1] * self.box[2]
        if shape_ids.dtype.is_floating_point or shape_ids.dtype == torch.bool or shape_ids.dim() != 1 \
                or shape_ids.numel() != self.Nz:
            raise ValueError(f"shape_ids must be a 1-D integer tensor of {self.Nz} zone ids for grid {self.grid}, "
                             f"got {shape_ids.dtype} {tuple(shape_ids.shape)}")
        self.shape_ids = shape_ids.contiguous().to(torch.int64)
        self.block_offset, self.block_id_of_tile, self.block_first_tile = _op("zone_layout", self.shape_ids)
        # the one host synchronisation of the path (the reference syncs here too,
        # dynamic_block_attention.py:153): N_b sizes the block tensors; the
        # kernel reports ids outside the candidate table as N_b = -1, before
        # any other kernel reads them
        self.N_b = int(self.block_offset[self.Nz].item())
        if self.N_b < 0:
            raise ValueError(f"shape_ids must index the {_CANDIDATES}-entry candidate table (0..{_CANDIDATES - 1})")


def rearrange_index(shape_ids: torch.Tensor, grid):
    _cuda(shape_ids)
    T, Hg, Wg = _grid(grid)
    lay = ZoneLayout(shape_ids, grid)  # validates the ids (count and range) before the kernel reads them
    return _op("rearrange_index", lay.shape_ids, [T, Hg, Wg])


def gather_pool(x: torch.Tensor, lay: ZoneLayout, valid: Optional[torch.Tensor] = None, *, rows: bool = True,
                pool: bool = False, counts: bool = False, dot_with: Optional[torch.Tensor] = None):
    """Rearrange x [B,H,S_in,D] (THW order of lay.box) into tile order (bf16
    rows [B,H,S,D] over lay.grid, padding rows zero) and optionally pool block
    means / counts / rowdot with dot_with.  Returns a dict."""
    _cuda(x, valid, dot_with)
    x = x.contiguous()
    B, H, S_in, D = x.shape
    if S_in != lay.S_in:
        raise ValueError(f"gather_pool: x has {S_in} tokens, the layout's input grid {lay.box} holds {lay.S_in}")
    S = lay.S
    _code(x)
    if dot_with is not None:
        dot_with = dot_with.contiguous()
        if dot_with.dtype != torch.bfloat16 or dot_with.shape != (B, H, S, D):
            raise ValueError("gather_pool: dot_with must be bf16 [B,H,S,D] in tile order")
    res = _op("gather_pool", x, _u8(valid), lay.shape_ids, lay.block_offset, list(lay.grid), list(lay.box), lay.N_b,
              rows, pool, counts, dot_with)
    return _gathered(res, rows, pool, counts, dot_with is not None)


def _gathered(res, rows, pool, counts, rowdot):
    keys = ("rows", "block_mean", "block_count", "tile_count", "valid_re", "rowdot")
    want = (rows, pool, counts, counts, counts, rowdot)
    return {k: (t if w else None) for k, t, w in zip(keys, res, want)}


def scatter_rows(rows: torch.Tensor, lay: ZoneLayout, out_dtype: torch.dtype) -> torch.Tensor:
    """Tile-order bf16 rows [B,H,S,D] -> THW order [B,H,S_in,D] of lay.box."""
    _cuda(rows)
    rows = rows.contiguous()
    B, H, S, D = rows.shape
    if S != lay.S:
        raise ValueError(f"scatter_rows: {S} rows, the layout holds {lay.S}")
    code = F32 if out_dtype == torch.float32 else BF16 if out_dtype == torch.bfloat16 else None
    if code is None:
        raise TypeError(f"prism_amd: unsupported dtype {out_dtype} (float32 or bfloat16)")
    return _op("scatter_rows", rows, lay.shape_ids, list(lay.grid), list(lay.box), code)


class ChunkLayout:
    """Uniform chunk layout of one side (queries or keys) of the fixed-shape
    BSA (flash_attn_bsa_3d / flash_attn_bsa_cross, bsa_interface.py:1123-1392).

    The input grid (T, H, W) is padded up to multiples of the chunk (ct, ch, cw)
    and cut into chunks in (nt, nh, nw) order (rearrange_THW_to_3d_block,
    bsa_interface.py:1105-1109); a 1-D sequence is the grid (1, 1, S) with
    chunk (1, 1, chunk_size).  Rows per head are rounded up to a multiple of
    128 (the attention kernels process tile pairs); rows past the padded grid
    are padding.  Chunks hold 64 or 128 tokens (one or two kernel tiles)."""

    def __init__(self, grid, chunk, device, pgrid=None):
        T, H, W = _grid(grid)
        ct, ch, cw = (int(c) for c in chunk)
        if min(T, H, W, ct, ch, cw) <= 0:
            raise ValueError(f"empty grid {grid} or chunk {chunk}")
        self.csz = ct * ch * cw
        if self.csz not in (64, 128):
            raise ValueError(f"chunk {tuple(chunk)} holds {self.csz} tokens; the MI355X kernels take chunks "
                             "of 64 or 128 tokens")
        self.grid = (T, H, W)
        self.chunk = (ct, ch, cw)
        if pgrid is None:
            pgrid = (-(-T // ct) * ct, -(-H // ch) * ch, -(-W // cw) * cw)
        self.pgrid = _grid(pgrid)
        if any(p < g or p % c for p, g, c in zip(self.pgrid, self.grid, self.chunk)):
            raise ValueError(f"padded grid {self.pgrid} must cover {self.grid} in whole chunks {self.chunk}")
        self.S_in = T * H * W
        self.Sp = self.pgrid[0] * self.pgrid[1] * self.pgrid[2]
        self.rows = -(-self.Sp // 128) * 128
        self.N_b = self.Sp // self.csz
        self.Nt = self.rows // 64
        self.padded = self.Sp != self.S_in or self.rows != self.Sp
        tpb = self.csz // 64
        self.tiles_per_block = tpb
        # block b owns tiles [tpb b, tpb b + tpb); tiles past the last block
        # (row padding) point at the last block and get empty lists
        self.block_first_tile = torch.arange(self.N_b + 1, device=device, dtype=torch.int32) * tpb
        self.block_id_of_tile = torch.clamp(torch.arange(self.Nt, device=device, dtype=torch.int32) // tpb,
                                            max=self.N_b - 1)

    def args(self):
        return (*self.grid, *self.pgrid, *self.chunk, self.rows)


def chunk_gather_pool(x: torch.Tensor, lay: ChunkLayout, valid: Optional[torch.Tensor] = None, *, rows: bool = True,
                      pool: bool = False, counts: bool = False, dot_with: Optional[torch.Tensor] = None):
    """Rearrange x [B,H,S_in,D] (THW of lay.grid) into lay's chunk order
    (bf16 rows, lay.rows per head, zero rows at padding) and optionally pool
    chunk means / counts / rowdot with dot_with.  Returns a dict like
    gather_pool."""
    _cuda(x, valid, dot_with)
    x = x.contiguous()
    B, H, S, D = x.shape
    if S != lay.S_in:
        raise ValueError(f"sequence length {S} != grid {lay.grid} ({lay.S_in} tokens)")
    _code(x)
    if dot_with is not None:
        dot_with = dot_with.contiguous()
        if dot_with.dtype != torch.bfloat16 or dot_with.shape != (B, H, lay.rows, D):
            raise ValueError("chunk_gather_pool: dot_with must be bf16 [B,H,rows,D] in chunk order")
    vm = _u8(valid)
    if vm is not None and vm.numel() != lay.S_in:
        raise ValueError(f"valid mask has {vm.numel()} entries, grid {lay.grid} has {lay.S_in} tokens")
    res = _op("chunk_gather_pool", x, vm, list(lay.grid), list(lay.pgrid), list(lay.chunk), lay.rows, rows, pool,
              counts, dot_with)
    return _gathered(res, rows, pool, counts, dot_with is not None)


def chunk_scatter_rows(rows: torch.Tensor, lay: ChunkLayout, out_dtype: torch.dtype) -> torch.Tensor:
    """Chunk-order bf16 rows [B,H,lay.rows,D] -> THW rows [B,H,S_in,D] of
    out_dtype (padding dropped)."""
    _cuda(rows)
    rows = rows.contiguous()
    B, H, R, D = rows.shape
    if R != lay.rows:
        raise ValueError(f"rows per head {R} != layout rows {lay.rows}")
    code = F32 if out_dtype == torch.float32 else BF16 if out_dtype == torch.bfloat16 else None
    if code is None:
        raise TypeError(f"prism_amd: unsupported dtype {out_dtype} (float32 or bfloat16)")
    return _op("chunk_scatter_rows", rows, list(lay.grid), list(lay.pgrid), list(lay.chunk), code)


# ------------------------------------------------------------------ selection
def block_scores(qc: torch.Tensor, kc: torch.Tensor, block_count: Optional[torch.Tensor]) -> torch.Tensor:
    """[..., Nq, D] x [..., Nk, D] fp32 block means -> [..., Nq, Nk] fp32
    scores (keys with block_count 0 get -inf when block_count is given)."""
    _cuda(qc, kc, block_count)
    Nq, D = qc.shape[-2], qc.shape[-1]
    Nk = kc.shape[-2]
    BH = qc.numel() // (Nq * D)
    if kc.shape[-1] != D or kc.numel() != BH * Nk * D:
        raise ValueError("block_scores: q and k means must share batch dims and D")
    return _op("block_scores", qc.contiguous().float(), kc.contiguous().float(), block_count)


def cdf_threshold_fixed(p: float) -> int:
    """Smallest X with fl32(X) * 2^-60 >= fl32(p): the fixed-point form of the
    test "cumsum < p" (exact integer bisection on the host)."""
    import numpy as np
    pf = np.float32(p)
    if not pf > 0:
        raise ValueError("cdf_threshold must be positive")
    lo, hi = 0, 1 << 62
    scale = np.float32(2.0 ** -60)
    while lo < hi:
        mid = (lo + hi) // 2
        if np.float32(np.uint64(mid)) * scale >= pf:
            hi = mid
        else:
            lo = mid + 1
    return lo


def selection_params(N: int, sparsity: Optional[float], cdf_threshold: Optional[float]):
    """(mode, k_lo, ub) exactly as bsa_interface.py:235-304 derives them."""
    if sparsity is not None and cdf_threshold is None:
        k = int((1 - sparsity) * N)
        return 0, k, k
    if sparsity is None and cdf_threshold is not None:
        return 1, 1, min(N, int(cdf_threshold * N) + 1)
    if sparsity is not None and cdf_threshold is not None:
        kt = max(1, int((1 - sparsity) * N))
        return 2, kt, min(N, max(kt, int(cdf_threshold * N) + 1))
    raise ValueError("Either sparsity or cdf_threshold must be provided")


def select_tiles(scores: torch.Tensor, sparsity, cdf_threshold, sm_scale: float, block_first_tile: torch.Tensor,
                 tile_count: Optional[torch.Tensor], want_blocks: bool = False, tiles_per_block: int = 2):
    """Per-row selection + tile expansion.  scores: [..., Nq, N] fp32 (N key
    blocks of at most tiles_per_block tiles).
    Returns dict(tiles [rows, tcap] int32, ntiles [rows], sel_blocks, nsel, tcap)."""
    _cuda(scores, block_first_tile, tile_count)
    N = scores.shape[-1]
    rows = scores.numel() // N
    mode, k_lo, ub = selection_params(N, sparsity, cdf_threshold)
    width = min(k_lo, N) if mode == 0 else ub
    tcap = max(tiles_per_block * width, 1)
    thr = cdf_threshold_fixed(cdf_threshold) if mode != 0 else 0
    tiles, ntiles, sel, nsel = _op("select_tiles", scores.contiguous(), mode, k_lo, ub, float(sm_scale), thr,
                                   block_first_tile, tile_count, tcap, max(width, 1), bool(want_blocks))
    if not want_blocks:
        sel = nsel = None
    return dict(tiles=tiles, ntiles=ntiles, sel_blocks=sel, nsel=nsel, tcap=tcap, width=width)


def tile_rows(ntiles: torch.Tensor, block_id_of_tile: torch.Tensor, BH: int, Nt: int, N_b: int, tcap: int,
              q_tile_count: Optional[torch.Tensor] = None):
    """Per-query-tile list starts and lengths; tiles whose q_tile_count is 0
    (no valid query token) get empty lists."""
    _cuda(ntiles, block_id_of_tile, q_tile_count)
    return _op("tile_rows", ntiles, block_id_of_tile, q_tile_count, int(BH), int(Nt), int(N_b), int(tcap))


def transpose_lists(qstart: torch.Tensor, qlen: torch.Tensor, qcols: torch.Tensor, BH: int, Nt: int,
                    Ntk: Optional[int] = None):
    """Per-query-tile key lists (Nt query tiles per head, key tiles < Ntk,
    default Nt) -> per-key-tile ascending query lists."""
    _cuda(qstart, qlen, qcols)
    Ntq, Ntk = int(Nt), int(Nt if Ntk is None else Ntk)
    return _op("transpose_lists", qstart, qlen, qcols, int(BH), Ntq, Ntk)


def lists_to_csr(start: torch.Tensor, length: torch.Tensor, cols: torch.Tensor):
    """Compact CSR of per-row lists given as (start int64, len int32, cols
    int32) with rows anywhere in cols (the outputs of tile_rows over
    select_tiles, transpose_lists and pair_union): returns (offsets int32
    [rows + 1], entries int32 [max(nnz, 1)]), row r's entries at
    [offsets[r], offsets[r + 1]).  Memory O(nnz) instead of the producers'
    rows x capacity buffers; one host read of nnz.  Lists with no entry at
    all still get a one-element buffer (never read), so the attention entry
    points, which reject null list pointers, take them."""
    _cuda(start, length, cols)
    return _op("lists_to_csr", start, length, cols)


def csr_offsets(length: torch.Tensor):
    """First half of lists_to_csr: (offsets int32 [rows + 1], nnz int64 [1]),
    both on the device (no host read)."""
    _cuda(length)
    return _op("lists_csr_offsets", length)


def csr_fill(start: torch.Tensor, length: torch.Tensor, cols: torch.Tensor, offsets: torch.Tensor, nnz: int):
    """Second half of lists_to_csr: the entries [max(nnz, 1)] at csr_offsets'
    offsets (nnz read by the caller)."""
    _cuda(start, length, cols, offsets)
    return _op("lists_csr_fill", start, length, cols, offsets, int(nnz))


class DeferredCompaction:
    """Compaction of several (start, len, cols) lists into CSR with one host
    read for all of them.  add() launches a list's offsets on the current
    stream and copies its nnz into pinned host memory without waiting;
    finish() waits for those copies (their events, not the streams: work
    queued after them, such as an attention kernel, is not waited for), then
    fills every list's CSR entries on the current stream.  The entries and
    their order are the source lists'."""

    def __init__(self, n: int):
        self.host = torch.empty(n, dtype=torch.int64, pin_memory=True)
        self.offsets = [None] * n
        self.events = [None] * n

    def add(self, i: int, lists):
        off, total = csr_offsets(lists[1])
        self.host[i:i + 1].copy_(total, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self.offsets[i], self.events[i] = off, ev

    def finish(self, lists_seq):
        """lists_seq[i]: the lists added as i (slots never added are left out)."""
        for ev in self.events[:len(lists_seq)]:
            ev.synchronize()
        nnz = self.host.tolist()
        return [(*csr_lists(self.offsets[i]), csr_fill(*lists, self.offsets[i], nnz[i]))
                for i, lists in enumerate(lists_seq)]


def csr_lists(offsets: torch.Tensor):
    """(start int64 [rows], len int32 [rows]) of CSR offsets: the list form the
    pair, union and attention kernels take (entries unchanged)."""
    o = offsets.to(torch.int64)
    return o[:-1].contiguous(), (o[1:] - o[:-1]).to(torch.int32)


def select_csr(scores: torch.Tensor, sparsity, cdf_threshold, sm_scale: float, lay: "ZoneLayout",
               tile_count: Optional[torch.Tensor] = None, q_tile_count: Optional[torch.Tensor] = None):
    """Block selection as CSR per query tile (get_select_indices_* of
    bsa_interface.py:235-304 expanded to tiles, dynamic_block_attention.py
    :297-319): scores [BH, N_b, N_b] fp32 -> (offsets int32 [BH*Nt + 1], key
    tiles int32 [nnz]), each query tile's list ascending.  tile_count drops
    padded key tiles; q_tile_count gives query tiles without a valid token an
    empty list.  The dense-compat form is select_tiles + tile_rows."""
    BH = scores.shape[0]
    sel = select_tiles(scores, sparsity, cdf_threshold, sm_scale, lay.block_first_tile, tile_count)
    qstart, qlen = tile_rows(sel["ntiles"], lay.block_id_of_tile, BH, lay.Nt, lay.N_b, sel["tcap"], q_tile_count)
    return lists_to_csr(qstart, qlen, sel["tiles"].view(-1))


def transpose_csr(offsets: torch.Tensor, cols: torch.Tensor, BH: int, Nt: int, Ntk: Optional[int] = None):
    """CSR per query tile -> CSR per key tile (csr_transpose;
    create_indices_k_from_indices_q_varlen, bsa_interface.py:147-161): each key
    tile's ascending query tiles.  Returns (offsets int32 [BH*Ntk + 1],
    query tiles int32 [nnz])."""
    start, length = csr_lists(offsets)
    return lists_to_csr(*transpose_lists(start, length, cols, BH, Nt, Ntk))


# ------------------------------------------------------------------ attention
def pair_tiles(start: torch.Tensor, length: torch.Tensor, cols: torch.Tensor, Nt: int,
               col_tiles: Optional[int] = None) -> torch.Tensor:
    """Pairing of the rows (tiles) of each group of 8 tiles of a head that
    maximises the summed list overlap of the pairs.  Returns pairmap [rows]
    int32: pair p of a head is tiles (pairmap[2p], pairmap[2p+1])."""
    _cuda(start, length, cols)
    return _op("pair_tiles", start, length, cols, int(Nt), int(Nt if col_tiles is None else col_tiles))


# fraction of an attention launch's workgroups ordered longest-list-first
ORDER_TAIL = 0.25


def pair_order(ulen: torch.Tensor, group: int, tail_frac: Optional[float] = None) -> torch.Tensor:
    """Workgroup order of an attention launch over the pairs of ulen
    (prism_pair_order): the XCD group mapping for the first ids, the last
    tail_frac of them (at most 16384) longest work list first.  group: 64 for
    the forward and dQ kernels, 32 for dK/dV."""
    _cuda(ulen)
    n = ulen.numel()
    frac = ORDER_TAIL if tail_frac is None else tail_frac
    tail = min(n, 16384, int(n * frac))
    return _op("pair_order", ulen, int(group), tail)


def pair_union(start: torch.Tensor, length: torch.Tensor, cols: torch.Tensor, Nt: int,
               tmasks: Optional[torch.Tensor] = None, col_tiles: Optional[int] = None,
               pairmap: Optional[torch.Tensor] = None):
    """Sorted union of the lists of each row pair (2p, 2p+1), or of the tiles
    pairmap pairs, with membership flags (entry = tile << 3 | partial << 2 |
    in_second << 1 | in_first).  Nt: rows (tiles) per head; col_tiles: bound of
    the listed tiles (default Nt).  Returns (ustart [rows/2] int64,
    ulen [rows/2] int32, ucols int32)."""
    _cuda(start, length, cols, tmasks, pairmap)
    ucap = int(Nt if col_tiles is None else col_tiles)
    return _op("pair_union", start, length, cols, int(Nt), ucap, pairmap, tmasks)


def quad_union(start: torch.Tensor, length: torch.Tensor, cols: torch.Tensor, Nt: int,
               tmasks: Optional[torch.Tensor] = None, col_tiles: Optional[int] = None,
               pairmap: Optional[torch.Tensor] = None):
    """Sorted union of the lists of each row quad (4q .. 4q+3, or pairmap[4q + k]:
    two pairs of a group) with membership flags (entry = tile << 5 |
    partial << 4 | member bits).  Nt (tiles per head) a multiple of 4.
    Returns (ustart [rows/4] int64, ulen [rows/4] int32, ucols int32)."""
    _cuda(start, length, cols, tmasks, pairmap)
    ucap = int(Nt if col_tiles is None else col_tiles)
    return _op("quad_union", start, length, cols, int(Nt), ucap, pairmap, tmasks)


def tile_masks(valid: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    """[Nt*64] uint8/bool tile-order validity -> [Nt] 64-bit masks (int64 storage)."""
    if valid is None:
        return None
    _cuda(valid)
    return _op("tile_masks", _u8(valid))


def lse_to_m2(lse: torch.Tensor) -> torch.Tensor:
    _cuda(lse)
    return _op("lse_to_m2", lse.contiguous().float())


def _bf16(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16 (MFMA kernels)")
    return t.contiguous()


def _attn_shapes(q, k, v):
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    if k.shape != (B, H, Sk, D) or v.shape != k.shape:
        raise ValueError(f"attention shapes differ: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    return B, H, Sq, Sk, D


def bsa_fwd(q, k, v, tmasks, qunion, sm_scale: float, qpair: Optional[torch.Tensor] = None,
            qorder: Optional[torch.Tensor] = None):
    """q [B,H,Sq,D], k, v [B,H,Sk,D] bf16 tile order; qunion = pair_union of
    the per-query-tile key lists (with the pairing qpair, or None for
    neighbouring tiles) -> (o bf16, lse fp32 natural)."""
    _cuda(q, k, v, tmasks, qpair, qorder)
    q, k, v = _bf16(q, "q"), _bf16(k, "k"), _bf16(v, "v")
    B, H, Sq, Sk, D = _attn_shapes(q, k, v)
    ustart, ulen, ucols = qunion
    return _op("bsa_fwd", q, k, v, tmasks, ustart, ulen, ucols, qpair, qorder, float(sm_scale))


def bsa_fwd_quad(q, k, v, tmasks, quadunion, sm_scale: float, quadmap: Optional[torch.Tensor] = None,
                 qorder: Optional[torch.Tensor] = None):
    """bsa_fwd over quad unions (quad_union of the per-query-tile key lists with
    the pairmap quadmap): the same o and lse, bit for bit, from one 8-wave
    workgroup per four query tiles.  Sq a multiple of 256."""
    _cuda(q, k, v, tmasks, quadmap, qorder)
    q, k, v = _bf16(q, "q"), _bf16(k, "k"), _bf16(v, "v")
    _attn_shapes(q, k, v)
    ustart, ulen, ucols = quadunion
    return _op("bsa_fwd_quad", q, k, v, tmasks, ustart, ulen, ucols, quadmap, qorder, float(sm_scale))


# dK/dV and dQ are independent: with BWD_CONCURRENT the dK/dV kernel runs on a
# second stream (default priority) so that the dQ kernel's workgroups fill the
# CUs that the end of the dK/dV launch leaves idle.  Measured 0.7% faster per
# step at config 4, but the two launches then overlap, so their individual
# durations no longer measure either kernel; off by default.
BWD_CONCURRENT = False
_side_streams: Dict[int, torch.cuda.Stream] = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    st = _side_streams.get(idx)
    if st is None:
        st = _side_streams[idx] = torch.cuda.Stream(device=idx)
    return st


# Side work that the attention launches do not depend on runs on the side
# stream while they run: the per-key-tile lists of the backward during the
# forward kernel (OVERLAP_SIDE_WORK), and, with OVERLAP_DKDV_SCATTER as well,
# the dK / dV scatters during the dQ kernel.  Inputs and outputs of the side
# work are recorded on the stream that did not allocate them (the caching
# allocator keeps their memory until that work is done).  The dQ launch keeps
# every CU busy until its work queue drains, so scatters queued beside it
# mostly wait for its end and then delay its last workgroups: off by default.
OVERLAP_SIDE_WORK = True
OVERLAP_DKDV_SCATTER = False

# The forward over quad unions (bsa_fwd_quad: four query tiles per staged K /
# V tile, bit-identical to bsa_fwd) when the query tiles per head are a
# multiple of 4; PRISM_QUADS=0 keeps the pair kernel.  dQ over the same quad
# unions (bsa_bwd_dq_quad, bit-identical to bsa_bwd_dq; the plan then keeps
# them for the backward): DQ_QUADS None (the default) takes it on the
# dynamic-shape path and not on the uniform and cross paths; True / False
# (PRISM_DQ_QUADS=1 / 0) force it either way.  The quads stage 42% fewer
# tile bytes but leave more wave slots idle (24% against 8% for pairs at
# config 4): forward 52.5 -> 49.7 ms there, dQ 59.6 -> 59.1 ms; on the
# uniform path (35% idle) forward 56.1-57.0 -> 52.1 ms but dQ 60.6-60.7 ->
# 61.5 ms.
QUADS = os.environ.get("PRISM_QUADS", "1") not in ("", "0")
_dq_env = os.environ.get("PRISM_DQ_QUADS", "")
DQ_QUADS: Optional[bool] = None if _dq_env == "" else _dq_env != "0"


def side_launch(device: torch.device, fn, reads=(), produces=None):
    """Run fn() on the side stream after the work queued so far on the
    current stream; returns (fn's result, event marking its end).  `reads`:
    current-stream tensors fn reads; `produces(result)`: the side-stream
    tensors the current stream will use."""
    main = torch.cuda.current_stream()
    side = _side_stream(device)
    side.wait_stream(main)
    with torch.cuda.stream(side):
        out = fn()
        done = torch.cuda.Event()
        done.record(side)
    for t in reads:
        if t is not None:
            t.record_stream(side)
    for t in (produces(out) if produces is not None else ()):
        if t is not None:
            t.record_stream(main)
    return out, done


def bsa_bwd(q, k, v, do, m2, delta, kv_valid, tmasks, qunion, kunion, sm_scale: float,
            qpair: Optional[torch.Tensor] = None, kpair: Optional[torch.Tensor] = None,
            qorder: Optional[torch.Tensor] = None, korder: Optional[torch.Tensor] = None, after_dkdv=None,
            q_quads: bool = False):
    """Backward over tile-order bf16 tensors; qunion / kunion = pair unions of
    the per-query-tile key lists and of the per-key-tile query lists, built
    with the pairings qpair / kpair (None: neighbouring tiles).  With q_quads,
    qunion is the quad_union of the per-query-tile lists (quadmap qpair,
    launch order qorder over quads) and dQ runs over quads (bit-identical).
    Returns dq, dk, dv (bf16, tile order).  after_dkdv(dk, dv), if given, is
    called between the dK/dV and the dQ launches."""
    _cuda(q, k, v, do, m2, delta, kv_valid, tmasks, qpair, kpair, qorder, korder)
    q, k, v, do = _bf16(q, "q"), _bf16(k, "k"), _bf16(v, "v"), _bf16(do, "do")
    B, H, Sq, Sk, D = _attn_shapes(q, k, v)
    if do.shape != q.shape:
        raise ValueError("do must have q's shape")
    def dkdv():
        return _op("bsa_bwd_dkdv", q, k, v, do, m2, delta, kv_valid, kunion[0], kunion[1], kunion[2], kpair, korder,
                   float(sm_scale))

    main = torch.cuda.current_stream()
    if BWD_CONCURRENT:
        side = _side_stream(q.device)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            dk, dv = dkdv()
        # the side stream reads and writes these: the allocator must not hand
        # their memory out again before its work is done
        for t in (q, k, v, do, m2, delta, kv_valid, kunion[0], kunion[1], kunion[2], kpair, korder, dk, dv):
            if t is not None:
                t.record_stream(side)
    else:
        dk, dv = dkdv()
    if after_dkdv is not None:
        after_dkdv(dk, dv)
    dq = _op("bsa_bwd_dq_quad" if q_quads else "bsa_bwd_dq", q, k, v, do, m2, delta, tmasks, qunion[0], qunion[1],
             qunion[2], qpair, qorder, float(sm_scale))
    if BWD_CONCURRENT:
        main.wait_stream(side)
    return dq, dk, dv


def bwd_preprocess(o: torch.Tensor, do: torch.Tensor) -> torch.Tensor:
    """delta = rowsum(o * do) over the last dim (bf16 inputs, fp32 out)."""
    _cuda(o, do)
    return _op("bwd_preprocess", _bf16(o, "o"), _bf16(do, "do"))
