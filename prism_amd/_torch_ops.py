"""Loads libprism_torch.so (TORCH_LIBRARY(prism): the C-ABI of
include/prism_bsa.h as PyTorch operators, torch.ops.prism.*) and registers
the fake (meta) implementation of every operator, so that shape propagation,
torch.compile tracing and torch.library.opcheck see the outputs' shapes and
dtypes without running a kernel.

The operator library is the only compute path of prism_amd.ops: if it is
missing the import fails loudly (there is no CPU or eager fallback).
"""
from __future__ import annotations

import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libprism_torch.so")
_loaded = False
_lock = threading.Lock()


def load():
    """Load the operator library once; returns torch.ops.prism."""
    global _loaded
    if _loaded:
        return torch.ops.prism
    with _lock:
        if not _loaded:
            if not os.path.exists(LIB_PATH):
                raise ImportError(f"{LIB_PATH} not found: build it first (python prism_amd/build.py); "
                                  "prism_amd has no fallback path")
            torch.ops.load_library(LIB_PATH)
            _register_fakes()
            _loaded = True
    return torch.ops.prism


def _empty(like, shape, dtype):
    return like.new_empty(shape, dtype=dtype)


def _none(like):
    return like.new_empty((0,), dtype=torch.float32)


def _zones(grid):
    return (grid[0] // 8) * (grid[1] // 8) * (grid[2] // 8)


def _register_fakes():
    def reg(qualname):
        # a library built before an operator was added lacks it: calling it
        # then fails loudly; its fake is simply not registered
        if not hasattr(torch.ops.prism, qualname.split("::")[1]):
            return lambda fn: fn
        return torch.library.register_fake(qualname)
    f32, bf16, u8, i32, i64 = torch.float32, torch.bfloat16, torch.uint8, torch.int32, torch.int64

    @reg("prism::zone_stats")
    def _(v, valid, grid, box):
        nz = _zones(grid)
        return _empty(v, (nz, 25 * v.shape[3]), f32), _empty(v, (nz, 24), u8)

    @reg("prism::audio_zone_stats")
    def _(norms, valid, grid, box):
        nz = _zones(grid)
        return _empty(norms, (nz,), f32), _empty(norms, (nz, 3), f32)

    @reg("prism::zone_gradient")
    def _(packed, axis_valid, D):
        nz = packed.shape[0]
        return _empty(packed, (nz,), f32), _empty(packed, (nz, 3), f32)

    @reg("prism::zone_shapes")
    def _(rho_raw, aniso, abar, vhat, method, lambda_a, tau_128, lambda_128):
        nz = rho_raw.shape[0]
        return _empty(rho_raw, (nz, 3), f32), _empty(rho_raw, (nz,), f32), _empty(rho_raw, (nz,), i64)

    @reg("prism::assign_shapes")
    def _(g, rho, method, tau_128, lambda_128):
        return _empty(g, (rho.shape[0],), i64)

    @reg("prism::a2v_norms")
    def _(residual):
        return _empty(residual, (residual.shape[0],), residual.dtype)

    @reg("prism::linear_rownorm")
    def _(x, weight, bias, norms_dtype):
        return _empty(x, (x.shape[0], weight.shape[0]), x.dtype), _empty(x, (x.shape[0],), f32 if norms_dtype == 0 else bf16)

    @reg("prism::zone_layout")
    def _(shape_ids):
        nz = shape_ids.numel()
        return _empty(shape_ids, (nz + 1,), i32), _empty(shape_ids, (nz * 8,), i32), _empty(shape_ids, (nz * 8 + 1,), i32)

    @reg("prism::rearrange_index")
    def _(shape_ids, grid):
        s = grid[0] * grid[1] * grid[2]
        return _empty(shape_ids, (s,), i64), _empty(shape_ids, (s,), i64)

    def gathered(x, S_out, N_b, rows, pool, counts, dot_with):
        B, H, D = x.shape[0], x.shape[1], x.shape[3]
        return (_empty(x, (B, H, S_out, D), bf16) if rows else _none(x),
                _empty(x, (B, H, N_b, D), f32) if pool else _none(x),
                _empty(x, (N_b,), i32) if counts else _none(x),
                _empty(x, (S_out // 64,), i32) if counts else _none(x),
                _empty(x, (S_out,), u8) if counts else _none(x),
                _empty(x, (B, H, S_out), f32) if dot_with is not None else _none(x))

    @reg("prism::gather_pool")
    def _(x, valid, shape_ids, block_offset, grid, box, N_b, rows, pool, counts, dot_with):
        return gathered(x, grid[0] * grid[1] * grid[2], N_b, rows, pool, counts, dot_with)

    @reg("prism::scatter_rows")
    def _(rows, shape_ids, grid, box, out_dtype):
        return _empty(rows, (rows.shape[0], rows.shape[1], box[0] * box[1] * box[2], rows.shape[3]),
                      f32 if out_dtype == 0 else bf16)

    @reg("prism::chunk_gather_pool")
    def _(x, valid, grid, pgrid, chunk, S_out, rows, pool, counts, dot_with):
        N_b = pgrid[0] * pgrid[1] * pgrid[2] // (chunk[0] * chunk[1] * chunk[2])
        return gathered(x, S_out, N_b, rows, pool, counts, dot_with)

    @reg("prism::chunk_scatter_rows")
    def _(rows, grid, pgrid, chunk, out_dtype):
        return _empty(rows, (rows.shape[0], rows.shape[1], grid[0] * grid[1] * grid[2], rows.shape[3]),
                      f32 if out_dtype == 0 else bf16)

    @reg("prism::block_scores")
    def _(qc, kc, block_count):
        return _empty(qc, (*qc.shape[:-1], kc.shape[-2]), f32)

    @reg("prism::select_tiles")
    def _(scores, mode, k_lo, ub, scale, thr, block_first_tile, tile_count, tcap, bcap, want_blocks):
        rows = scores.numel() // scores.shape[-1]
        return (_empty(scores, (rows, tcap), i32), _empty(scores, (rows,), i32),
                _empty(scores, (rows, bcap), i32) if want_blocks else _none(scores),
                _empty(scores, (rows,), i32) if want_blocks else _none(scores))

    @reg("prism::tile_rows")
    def _(ntiles, block_id_of_tile, q_tile_count, BH, Nt, N_b, tcap):
        return _empty(ntiles, (BH * Nt,), i64), _empty(ntiles, (BH * Nt,), i32)

    @reg("prism::transpose_lists")
    def _(qstart, qlen, qcols, BH, Ntq, Ntk):
        return _empty(qstart, (BH * Ntk,), i64), _empty(qstart, (BH * Ntk,), i32), _empty(qstart, (BH * Ntk * Ntq,), i32)

    @reg("prism::pair_tiles")
    def _(start, length, cols, row_tiles, col_tiles):
        return _empty(start, (start.numel(),), i32)

    @reg("prism::pair_union")
    def _(start, length, cols, row_tiles, col_tiles, pairmap, tile_masks):
        pairs = start.numel() // 2
        return (_empty(start, (pairs,), i64), _empty(start, (pairs,), i32),
                _empty(start, (max(pairs * col_tiles, 1),), i32))

    @reg("prism::quad_union")
    def _(start, length, cols, row_tiles, col_tiles, pairmap, tile_masks):
        quads = start.numel() // 4
        return (_empty(start, (quads,), i64), _empty(start, (quads,), i32),
                _empty(start, (max(quads * col_tiles, 1),), i32))

    @reg("prism::pair_order")
    def _(ulen, group, tail):
        return _empty(ulen, (ulen.numel(),), i32)

    @reg("prism::lists_to_csr")
    def _(start, length, cols):
        nnz = torch.library.get_ctx().new_dynamic_size(min=1)  # max(entries, 1): never an empty buffer
        return _empty(start, (start.numel() + 1,), i32), _empty(start, (nnz,), i32)

    @reg("prism::lists_csr_offsets")
    def _(length):
        return _empty(length, (length.numel() + 1,), i32), _empty(length, (1,), i64)

    @reg("prism::lists_csr_fill")
    def _(start, length, cols, offsets, nnz):
        return _empty(start, (max(nnz, 1),), i32)

    @reg("prism::tile_masks")
    def _(valid):
        return _empty(valid, (valid.numel() // 64,), i64)

    @reg("prism::lse_to_m2")
    def _(lse):
        return _empty(lse, lse.shape, f32)

    @reg("prism::bsa_fwd")
    def _(q, k, v, tile_masks, ustart, ulen, ucols, pairmap, order, sm_scale):
        return _empty(q, q.shape, q.dtype), _empty(q, q.shape[:3], f32)

    @reg("prism::bsa_fwd_quad")
    def _(q, k, v, tile_masks, ustart, ulen, ucols, quadmap, order, sm_scale):
        return _empty(q, q.shape, q.dtype), _empty(q, q.shape[:3], f32)

    @reg("prism::bwd_preprocess")
    def _(o, do):
        return _empty(o, o.shape[:-1], f32)

    @reg("prism::bsa_bwd_dkdv")
    def _(q, k, v, do, m2, delta, kv_valid, ustart, ulen, ucols, pairmap, order, sm_scale):
        return _empty(k, k.shape, k.dtype), _empty(v, v.shape, v.dtype)

    @reg("prism::bsa_bwd_dq")
    def _(q, k, v, do, m2, delta, tile_masks, ustart, ulen, ucols, pairmap, order, sm_scale):
        return _empty(q, q.shape, q.dtype)

    @reg("prism::bsa_bwd_dq_quad")
    def _(q, k, v, do, m2, delta, tile_masks, ustart, ulen, ucols, quadmap, order, sm_scale):
        return _empty(q, q.shape, q.dtype)
