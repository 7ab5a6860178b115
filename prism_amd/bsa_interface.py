"""Kernel-level API of the block-sparse attention path, MI355X implementation.

Mirrors the functions of hymm/models/modules/block_sparse_attention/bsa_interface.py
(names, argument meaning, return layout), backed by libprism_bsa.so:
  * the helpers the dynamic path uses: cal_score, the three selection
    helpers, attn_fwd_bsa_varlen / attn_bwd_bsa_varlen over given per-tile
    lists (64-token tiles, the "align" variant the dynamic path reaches,
    dynamic_block_attention.py:322-326; other chunk sizes raise ValueError),
    create_indices_k_from_indices_q_varlen;
  * the uniform-shape entry points flash_attn_bsa, flash_attn_bsa_3d and
    flash_attn_bsa_cross (prism_amd.uniform_block_attention; chunks of 64 or
    128 tokens).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import ops
from .uniform_block_attention import flash_attn_bsa, flash_attn_bsa_3d, flash_attn_bsa_cross  # noqa: F401


def cal_score(q: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
    """Block-level scores q k^T in fp32 (bsa_interface.py:203-207; the
    reference returns q's dtype)."""
    return ops.block_scores(q, k, None)


def _identity_first_tile(N: int, device) -> torch.Tensor:
    return torch.arange(N + 1, device=device, dtype=torch.int32)


def _select_blocks(score: torch.Tensor, sparsity, cdf_threshold, sm_scale):
    N = score.shape[-1]
    res = ops.select_tiles(score.float(), sparsity, cdf_threshold, sm_scale if sm_scale is not None else 1.0,
                           _identity_first_tile(N, score.device), None, want_blocks=True)
    lead = score.shape[:-1]
    idx = res["sel_blocks"].view(*lead, -1).to(torch.int64)
    lens = res["nsel"].view(*lead)
    return idx, lens


def get_select_indices_topk_from_score(score: torch.Tensor, sparsity: float):
    """k = int((1 - sparsity) N) largest scores per row, ascending indices
    (bsa_interface.py:235-248).  Returns (indices [..., k] int64, lens int32)."""
    return _select_blocks(score, sparsity, None, None)


def get_select_indices_cdf_from_score(score: torch.Tensor, cdf_threshold: float, sm_scale: float):
    """Smallest prefix of the softmax-sorted blocks reaching cdf_threshold
    (bsa_interface.py:257-275).  Slots past the count hold the sentinel N;
    lens counts the valid entries."""
    return _select_blocks(score, None, cdf_threshold, sm_scale)


def get_select_indices_cdf_topk_from_score(score: torch.Tensor, sparsity: float, cdf_threshold: float,
                                           sm_scale: float):
    """Hybrid: max(top-k, cdf prefix) (bsa_interface.py:284-304)."""
    return _select_blocks(score, sparsity, cdf_threshold, sm_scale)


def _lists_from_dense(block_indices: torch.Tensor, block_indices_lens: torch.Tensor):
    B, H, M, W = block_indices.shape
    qcols = block_indices.to(torch.int32).contiguous().view(-1)
    qstart = torch.arange(B * H * M, device=block_indices.device, dtype=torch.int64) * W
    qlen = block_indices_lens.to(torch.int32).contiguous().view(-1)
    return qstart, qlen, qcols


def _check_chunks(chunk_size_q, chunk_size_k):
    if chunk_size_q != 64 or chunk_size_k != 64:
        raise ValueError(f"only 64x64 tiles are implemented (got chunk_size_q={chunk_size_q}, "
                         f"chunk_size_k={chunk_size_k})")


def attn_fwd_bsa_varlen(q, k, v, sm_scale, block_indices, block_indices_lens, chunk_size_q=64, chunk_size_k=64,
                        sparsity=None, kv_valid_mask: Optional[torch.Tensor] = None):
    """Block-sparse attention forward over per-query-tile key-tile lists
    (attn_fwd_bsa_varlen_triton, bsa_interface.py:328-385).  q, k, v: [B,H,S,D]
    bf16; block_indices [B,H,S/64,W], block_indices_lens [B,H,S/64].
    Returns (o [B,H,S,D], lse [B,H,S] natural log)."""
    _check_chunks(chunk_size_q, chunk_size_k)
    qstart, qlen, qcols = _lists_from_dense(block_indices, block_indices_lens)
    Ntq, Ntk = q.shape[2] // 64, k.shape[2] // 64
    tm = ops.tile_masks(ops._u8(kv_valid_mask))
    if ops.QUADS and Ntq % 4 == 0:
        # four query tiles per staged K / V tile (two overlap pairs of each
        # group of 8), the same outputs bit for bit
        qpair = ops.pair_tiles(qstart, qlen, qcols, Ntq, Ntk)
        quad = ops.quad_union(qstart, qlen, qcols, Ntq, tm, col_tiles=Ntk, pairmap=qpair)
        return ops.bsa_fwd_quad(q, k, v, tm, quad, sm_scale, qpair, ops.pair_order(quad[1], 32))
    qunion = ops.pair_union(qstart, qlen, qcols, Ntq, tm, col_tiles=Ntk)
    return ops.bsa_fwd(q, k, v, tm, qunion, sm_scale)


def create_indices_k_from_indices_q_varlen(block_indices: torch.Tensor, N_cols_mask: int):
    """Per-key-tile ascending query lists (bsa_interface.py:147-161).
    Returns ([B,H,N_cols,M] padded with M, lens [B,H,N_cols])."""
    B, H, M, W = block_indices.shape
    N = int(N_cols_mask)
    lens = (block_indices < N).sum(-1).to(torch.int32)
    qstart, qlen, qcols = _lists_from_dense(block_indices, lens)
    kstart, klen, kcols = ops.transpose_lists(qstart, qlen, qcols, B * H, M, N)
    kc = kcols.view(B, H, N, M)
    pos = torch.arange(M, device=kc.device).view(1, 1, 1, M)
    kc = torch.where(pos < klen.view(B, H, N, 1), kc, torch.full_like(kc, M)).to(torch.int64)
    return kc, klen.view(B, H, N)


def attn_bwd_bsa_varlen(do, q, k, v, o, dq, dk, dv, sm_scale, lse, block_indices, block_indices_lens,
                        chunk_size_q=64, chunk_size_k=64, sparsity=None, kv_valid_mask=None):
    """Backward of attn_fwd_bsa_varlen; writes dq, dk, dv in place
    (attn_bwd_bsa_varlen_triton, bsa_interface.py:387-523).  lse is the
    natural-log LSE returned by the forward."""
    _check_chunks(chunk_size_q, chunk_size_k)
    B, H, S, D = q.shape
    Ntq, Ntk = S // 64, k.shape[2] // 64
    qstart, qlen, qcols = _lists_from_dense(block_indices, block_indices_lens)
    do = do.to(torch.bfloat16).contiguous()
    o = o.to(torch.bfloat16).contiguous()
    delta = ops.bwd_preprocess(o, do)
    klists = ops.transpose_lists(qstart, qlen, qcols, B * H, Ntq, Ntk)
    kv = ops._u8(kv_valid_mask)
    tm = ops.tile_masks(kv)
    qunion = ops.pair_union(qstart, qlen, qcols, Ntq, tm, col_tiles=Ntk)
    kunion = ops.pair_union(*klists, Ntk, None, col_tiles=Ntq)
    m2 = ops.lse_to_m2(lse)
    g_q, g_k, g_v = ops.bsa_bwd(q, k, v, do, m2, delta, kv, tm, qunion, kunion, sm_scale)
    dq.copy_(g_q)
    dk.copy_(g_k)
    dv.copy_(g_v)
    return dq, dk, dv


__all__ = [
    "cal_score", "get_select_indices_topk_from_score", "get_select_indices_cdf_from_score",
    "get_select_indices_cdf_topk_from_score", "attn_fwd_bsa_varlen", "attn_bwd_bsa_varlen",
    "create_indices_k_from_indices_q_varlen", "flash_attn_bsa", "flash_attn_bsa_3d", "flash_attn_bsa_cross",
]
