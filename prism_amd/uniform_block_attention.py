"""Fixed-chunk-shape block-sparse attention (uniform BSA), MI355X implementation.

Drop-in for the uniform-shape path of
hymm/models/modules/block_sparse_attention/bsa_interface.py of the reference:

  flash_attn_bsa        _attention_bsa.apply (bsa_interface.py:597-683): q, k, v
                        already in chunk order, chunk sizes in tokens;
  flash_attn_bsa_3d     (:1123-1176): THW video tokens cut into 3-D chunks;
  flash_attn_bsa_cross  (:1276-1392): asymmetric 3-D / 1-D query and key
                        sequences (e.g. audio queries over video keys), padded
                        internally to whole chunks.

All three share one engine.  Each side (queries, keys) has a ChunkLayout;
one gather kernel per tensor does the padding, the chunk rearrangement and the
(masked) chunk mean pooling in a single pass (the reference runs F.pad, a
permute copy and a separate pooling pass); scores, selection, list building
and attention are the kernels of the dynamic path (prism_block_scores,
prism_select_tiles, prism_pair_union, prism_bsa_fwd / _bwd_*), which accept
query and key sequences of different lengths; one scatter kernel per output
undoes the rearrangement and drops the padding.

Deliberate differences from the reference, as in the dynamic path: chunk means
and scores are fp32 with one fixed summation order (the reference pools and
scores in q's dtype); with compute_padded_queries=False (the adapters and
flash_attn_bsa_cross, which slice padded rows away) query tiles with no valid
token get empty lists (their output rows are 0 instead of attention over the
selected keys), while flash_attn_bsa and flash_attn_bsa_3d attend for them by
default, as the reference does; queries are pooled with their own validity in
their own chunk order (the reference pools them with the key-order mask, which
is the same thing whenever the two chunk shapes agree).
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch

from . import ops


class _ChunkPlan:
    """Rearranged rows, selection and work lists of one call (built under no_grad)."""

    def __init__(self, q, k, v, lq: ops.ChunkLayout, lk: ops.ChunkLayout, q_valid, k_valid, sparsity,
                 cdf_threshold, sm_scale, compute_padded_queries=False, keep_scores=False, compact_lists=False):
        B, H, _, D = q.shape
        BH = B * H
        self.lq, self.lk = lq, lk
        self.B, self.H, self.D = B, H, D
        gq = ops.chunk_gather_pool(q, lq, q_valid, rows=True, pool=True, counts=True)
        gk = ops.chunk_gather_pool(k, lk, k_valid, rows=True, pool=True, counts=True)
        gv = ops.chunk_gather_pool(v, lk, None, rows=True)
        self.q_re, self.k_re, self.v_re = gq["rows"], gk["rows"], gv["rows"]
        q_masked = q_valid is not None or lq.padded
        k_masked = k_valid is not None or lk.padded
        self.kv_valid = gk["valid_re"] if k_masked else None
        # uniform path: no invalid-key fill of the scores (bsa_interface.py:611-631)
        scores = ops.block_scores(gq["block_mean"].view(BH, lq.N_b, D), gk["block_mean"].view(BH, lk.N_b, D), None)
        sel = ops.select_tiles(scores, sparsity, cdf_threshold, sm_scale, lk.block_first_tile,
                               gk["tile_count"] if k_masked else None, tiles_per_block=lk.tiles_per_block)
        # scores are freed once the lists exist (kept only on request)
        self.scores = scores if keep_scores else None
        del scores
        self.sel = sel
        if q_masked and not compute_padded_queries:
            qcount = gq["tile_count"]  # tiles without a valid query token (and row padding) get no list
        elif lq.rows != lq.Sp:
            qcount = (torch.arange(lq.Nt, device=q.device) < lq.Sp // 64).to(torch.int32)  # row padding only
        else:
            qcount = None
        self.qstart, self.qlen = ops.tile_rows(sel["ntiles"], lq.block_id_of_tile, BH, lq.Nt, lq.N_b, sel["tcap"],
                                               qcount)
        self.qcols = sel["tiles"].view(-1)
        # compact lists: the pair unions the backward keeps as CSR, O(nnz)
        # memory (settle(); one host read of both nnz; same entries)
        self.compact = compact_lists
        self._settled = False
        self.tmasks = ops.tile_masks(self.kv_valid) if k_masked else None
        self.qpair = ops.pair_tiles(self.qstart, self.qlen, self.qcols, lq.Nt, lk.Nt)
        self.qunion = ops.pair_union(self.qstart, self.qlen, self.qcols, lq.Nt, self.tmasks, col_tiles=lk.Nt,
                                     pairmap=self.qpair)
        self._csr = ops.DeferredCompaction(3) if compact_lists else None
        if compact_lists:
            self._csr.add(0, self.qunion)
        # launch order of the forward and dQ kernels (longest lists last-dispatched first)
        self.qorder = ops.pair_order(self.qunion[1], 64)
        # quad unions (two pairs per workgroup), which the forward and dQ
        # kernels walk instead of the pair unions when ops.QUADS is set (same
        # results, bit for bit)
        self.qquad = self.qquad_order = self.qquadmap = None
        # dq_quads: dQ walks them too (only when ops.DQ_QUADS forces it on
        # these paths, whose quads leave more slots idle), so the backward
        # keeps them
        self.quads = ops.QUADS and lq.Nt % 4 == 0
        self.dq_quads = self.quads and ops.DQ_QUADS is True
        if self.quads:
            self.qquadmap = self.qpair
            self.qquad = ops.quad_union(self.qstart, self.qlen, self.qcols, lq.Nt, self.tmasks, col_tiles=lk.Nt,
                                        pairmap=self.qquadmap)
            if compact_lists and self.dq_quads:
                self._csr.add(2, self.qquad)
            self.qquad_order = ops.pair_order(self.qquad[1], 32)
        self.klists = None
        self.kpair = None
        self.kunion = None
        self.korder = None
        self.keys_ready = None  # event of a key-list build on the side stream

    def key_lists_side(self):
        """key_lists on the side stream, after the work queued so far on the
        current stream."""
        if self.kunion is not None:
            return
        _, self.keys_ready = ops.side_launch(
            self.qcols.device, self.key_lists, reads=(self.qstart, self.qlen, self.qcols),
            produces=lambda _: (*self.klists, self.kpair, *self.kunion, self.korder,
                                self._csr.offsets[1] if self._csr is not None else None))

    def join_side(self):
        """Make the current stream wait for a side-stream key-list build (the
        fork is joined in the forward that opened it)."""
        if getattr(self, "keys_ready", None) is not None:
            torch.cuda.current_stream().wait_event(self.keys_ready)
            self.keys_ready = None

    def key_lists(self):
        self.join_side()
        if self.kunion is None:
            self.klists = ops.transpose_lists(self.qstart, self.qlen, self.qcols, self.B * self.H, self.lq.Nt,
                                              self.lk.Nt)
            self.kpair = ops.pair_tiles(*self.klists, self.lk.Nt, self.lq.Nt)
            self.kunion = ops.pair_union(*self.klists, self.lk.Nt, None, col_tiles=self.lq.Nt, pairmap=self.kpair)
            self.korder = ops.pair_order(self.kunion[1], 32)
            if self._csr is not None:
                self._csr.add(1, self.kunion)
        return self.kunion

    def settle(self):
        """Keep only what the backward reads: the pair unions, and the quad
        unions when dQ walks them (compact CSR when the plan is compact, one
        batched host read of their nnz), pairings and launch orders; the
        per-tile lists and the forward-only quad unions are released."""
        if self._settled:
            return
        self.key_lists()
        if self._csr is not None:
            lists = [self.qunion, self.kunion] + ([self.qquad] if self.dq_quads else [])
            done = self._csr.finish(lists)
            self.qunion, self.kunion = done[:2]
            if self.dq_quads:
                self.qquad = done[2]
            self._csr = None
        if not self.dq_quads:  # the forward's only: released once it is queued
            self.qquad = self.qquad_order = None
        self.qcols = None
        self.klists = None
        self.sel = {key: val for key, val in self.sel.items() if key != "tiles"}
        self._settled = True

    def sum_lens(self) -> int:
        """Executed (query tile, key tile) pairs (host sync)."""
        return int(self.qlen.sum().item())


class _ChunkBSA(torch.autograd.Function):
    """Attention over a _ChunkPlan with gradients to the input q, k, v
    (_attention_bsa.forward / backward, bsa_interface.py:641-681, plus the
    autograd of the rearrangements :1162-1175)."""

    @staticmethod
    def forward(ctx, q, k, v, plan: _ChunkPlan, sm_scale: float):
        grads = any(ctx.needs_input_grad[:3])
        if grads:
            # the backward's lists, beside the forward kernel (or before it)
            if ops.OVERLAP_SIDE_WORK:
                plan.key_lists_side()
            else:
                plan.key_lists()
        if plan.qquad is not None:
            o_re, lse = ops.bsa_fwd_quad(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qquad, sm_scale,
                                         plan.qquadmap, plan.qquad_order)
        else:
            o_re, lse = ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qunion, sm_scale, plan.qpair,
                                    plan.qorder)
        plan.join_side()  # queued after the forward kernel: the key lists still run beside it
        if grads:
            plan.settle()  # release the per-tile lists; compact the unions while the forward runs
        ctx.plan = plan
        ctx.sm_scale = sm_scale
        ctx.in_dtypes = (q.dtype, k.dtype, v.dtype)
        ctx.save_for_backward(o_re, lse)
        return ops.chunk_scatter_rows(o_re, plan.lq, q.dtype)

    @staticmethod
    def backward(ctx, do):
        plan: _ChunkPlan = ctx.plan
        o_re, lse = ctx.saved_tensors
        gd = ops.chunk_gather_pool(do.contiguous(), plan.lq, None, rows=True, dot_with=o_re)
        kunion = plan.key_lists()
        m2 = ops.lse_to_m2(lse)
        tq, tk, tv = ctx.in_dtypes
        side = {}

        def scatter_dkdv(dk_re, dv_re):
            # dK and dV back to the input order on the side stream, during the dQ kernel
            if ops.OVERLAP_SIDE_WORK and ops.OVERLAP_DKDV_SCATTER:
                side["dkdv"] = ops.side_launch(
                    dk_re.device,
                    lambda: (ops.chunk_scatter_rows(dk_re, plan.lk, tk), ops.chunk_scatter_rows(dv_re, plan.lk, tv)),
                    reads=(dk_re, dv_re), produces=lambda out: out)

        quads = plan.dq_quads
        dq_re, dk_re, dv_re = ops.bsa_bwd(plan.q_re, plan.k_re, plan.v_re, gd["rows"], m2, gd["rowdot"],
                                          plan.kv_valid, plan.tmasks, plan.qquad if quads else plan.qunion, kunion,
                                          ctx.sm_scale, plan.qquadmap if quads else plan.qpair, plan.kpair,
                                          plan.qquad_order if quads else plan.qorder, plan.korder,
                                          after_dkdv=scatter_dkdv, q_quads=quads)
        dq = ops.chunk_scatter_rows(dq_re, plan.lq, tq)
        if "dkdv" in side:
            (dk, dv), done = side["dkdv"]
            torch.cuda.current_stream().wait_event(done)
        else:
            dk = ops.chunk_scatter_rows(dk_re, plan.lk, tk)
            dv = ops.chunk_scatter_rows(dv_re, plan.lk, tv)
        return dq, dk, dv, None, None


def _check_qkv(q, k, v):
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be [B, H, S, D]")
    assert q.shape[-1] == k.shape[-1] and k.shape[-1] == v.shape[-1]
    assert q.shape[-1] in {16, 32, 64, 128, 256}
    if q.shape[-1] not in (64, 128):
        raise ValueError(f"head_dim {q.shape[-1]} unsupported by the MI355X kernels (64, 128)")
    if q.shape[:2] != k.shape[:2] or k.shape != v.shape:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")


def plan_chunked(q, k, v, lq: ops.ChunkLayout, lk: ops.ChunkLayout, *, sparsity, cdf_threshold, sm_scale,
                 q_valid=None, k_valid=None, compute_padded_queries=False, keep_scores=False,
                 compact_lists=False) -> _ChunkPlan:
    """Selection half of the uniform path (no attention).  keep_scores keeps
    the fp32 chunk scores on the plan (plan.scores) for inspection;
    compact_lists makes plan.settle() keep the pair unions in compact CSR
    form (O(nnz) memory)."""
    if sparsity is None and cdf_threshold is None:
        raise ValueError("Either sparsity or cdf_threshold must be provided")
    with torch.no_grad():
        return _ChunkPlan(q.detach(), k.detach(), v.detach(), lq, lk, q_valid, k_valid, sparsity, cdf_threshold,
                          sm_scale, compute_padded_queries, keep_scores, compact_lists)


def bsa_chunked(q, k, v, lq: ops.ChunkLayout, lk: ops.ChunkLayout, *, sparsity, cdf_threshold, sm_scale,
                q_valid=None, k_valid=None, compute_padded_queries=False, compact_lists=True) -> torch.Tensor:
    """Uniform BSA of q [B,H,Sq,D] (THW of lq.grid) over k, v [B,H,Sk,D] (THW
    of lk.grid); returns [B,H,Sq,D] in q's dtype and order."""
    plan = plan_chunked(q, k, v, lq, lk, sparsity=sparsity, cdf_threshold=cdf_threshold, sm_scale=sm_scale,
                        q_valid=q_valid, k_valid=k_valid, compute_padded_queries=compute_padded_queries,
                        compact_lists=compact_lists)
    return _ChunkBSA.apply(q, k, v, plan, sm_scale)


def flash_attn_bsa(q, k, v, chunk_size_q, chunk_size_k, sparsity, cdf_threshold, sm_scale, kv_valid_mask=None,
                   q_valid_mask=None, score_modifier=None, compute_padded_queries=True):
    """_attention_bsa.apply (bsa_interface.py:597-683): q, k, v [B,H,S,D]
    already in chunk order; chunk sizes in tokens (64 or 128).  The query
    chunks are pooled with q_valid_mask, else with kv_valid_mask when
    Sq == Sk (:606-611).  Returns [B,H,Sq,D] in chunk order."""
    _check_qkv(q, k, v)
    if score_modifier is not None:
        raise NotImplementedError("score_modifier (audio-guided score modulation) is not part of this build")
    Sq, Sk = q.shape[2], k.shape[2]
    lq = ops.ChunkLayout((1, 1, Sq), (1, 1, chunk_size_q), q.device)
    lk = ops.ChunkLayout((1, 1, Sk), (1, 1, chunk_size_k), q.device)
    q_valid = q_valid_mask
    if q_valid is None and kv_valid_mask is not None and Sq == Sk:
        q_valid = kv_valid_mask
    return bsa_chunked(q, k, v, lq, lk, sparsity=sparsity, cdf_threshold=cdf_threshold, sm_scale=sm_scale,
                       q_valid=q_valid, k_valid=kv_valid_mask, compute_padded_queries=compute_padded_queries)


def flash_attn_bsa_3d(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, latent_shape_q, latent_shape_k,
                      sparsity=0.875, cdf_threshold=None, chunk_3d_shape_q: Sequence[int] = (4, 4, 8),
                      chunk_3d_shape_k: Sequence[int] = (4, 4, 8), valid_mask: Optional[torch.Tensor] = None,
                      compute_padded_queries: bool = True) -> torch.Tensor:
    """Uniform 3-D-chunk BSA over THW tokens (bsa_interface.py:1123-1176).
    q: [B,H,Sq,D], k, v: [B,H,Sk,D] in THW order of latent_shape_q / _k, each a
    multiple of its chunk shape; valid_mask [Sq] (True = valid, Sq == Sk)
    masks padded keys and is excluded from the pooled means.  Returns
    [B,H,Sq,D] THW in q's dtype."""
    _check_qkv(q, k, v)
    Sq, Sk = q.shape[2], k.shape[2]
    Tq, Hq, Wq = latent_shape_q
    Tk, Hk, Wk = latent_shape_k
    assert Tq * Hq * Wq == Sq
    assert Tk * Hk * Wk == Sk
    tq, hq, wq = chunk_3d_shape_q
    tk, hk, wk = chunk_3d_shape_k
    assert Tq % tq == 0 and Hq % hq == 0 and Wq % wq == 0
    assert Tk % tk == 0 and Hk % hk == 0 and Wk % wk == 0
    if valid_mask is not None and Sq != Sk:
        raise ValueError("valid_mask needs Sq == Sk (it masks both sides)")
    lq = ops.ChunkLayout(latent_shape_q, chunk_3d_shape_q, q.device)
    lk = ops.ChunkLayout(latent_shape_k, chunk_3d_shape_k, q.device)
    sm_scale = 1.0 / (q.shape[-1] ** 0.5)
    return bsa_chunked(q, k, v, lq, lk, sparsity=sparsity, cdf_threshold=cdf_threshold, sm_scale=sm_scale,
                       q_valid=valid_mask, k_valid=valid_mask, compute_padded_queries=compute_padded_queries)


def _side_layout(structure: str, S: int, grid, chunk_3d, chunk_size: int, device, name: str) -> ops.ChunkLayout:
    if structure == "3d":
        assert grid is not None
        T, H, W = grid
        if T * H * W != S:
            raise ValueError(f"{name}_grid_size {tuple(grid)} does not hold {S} tokens")
        return ops.ChunkLayout(grid, chunk_3d or (4, 4, 4), device)
    if structure != "1d":
        raise ValueError(f"{name}_structure must be '3d' or '1d', got {structure!r}")
    return ops.ChunkLayout((1, 1, S), (1, 1, chunk_size), device)


def flash_attn_bsa_cross(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_structure: str, k_structure: str,
                         q_grid_size=None, k_grid_size=None, sparsity=0.875, cdf_threshold=None, chunk_size_q=64,
                         chunk_size_k=64, chunk_3d_shape_q=None, chunk_3d_shape_k=None) -> torch.Tensor:
    """Cross-modal BSA with asymmetric query / key structures
    (bsa_interface.py:1276-1392): each side is "3d" (THW tokens of its grid,
    3-D chunks, default 4x4x4) or "1d" (a sequence in chunks of chunk_size
    tokens) and is padded to whole chunks internally; padded keys are masked,
    padded tokens are excluded from the pooled means, and the output has q's
    original length and order."""
    _check_qkv(q, k, v)
    Sq, Sk = q.shape[2], k.shape[2]
    lq = _side_layout(q_structure, Sq, q_grid_size, chunk_3d_shape_q, chunk_size_q, q.device, "q")
    lk = _side_layout(k_structure, Sk, k_grid_size, chunk_3d_shape_k, chunk_size_k, q.device, "k")
    sm_scale = 1.0 / (q.shape[-1] ** 0.5)
    return bsa_chunked(q, k, v, lq, lk, sparsity=sparsity, cdf_threshold=cdf_threshold, sm_scale=sm_scale)


__all__ = ["flash_attn_bsa", "flash_attn_bsa_3d", "flash_attn_bsa_cross", "bsa_chunked", "plan_chunked"]
