"""Dynamic-block-shape block-sparse attention, MI355X implementation.

Drop-in for hymm/models/modules/block_sparse_attention/dynamic_block_attention.py
of the reference: ``flash_attn_bsa_3d_dynamic`` keeps its signature, return
contract, errors and autograd behaviour (gradients flow to q, k, v only).

Pipeline (all HIP kernels of libprism_bsa.so, one host sync for N_b):
  (1) zone statistics + shape ids      prism_zone_stats / _gradient / _shapes
  (2) zone layout (block/tile maps)    prism_zone_layout
  (3) rearranged rows + block means    prism_gather_pool (q, k, v)
  (4) fp32 block scores + selection    prism_block_scores, prism_select_tiles
  (5) tile lists per query tile        prism_tile_rows
  (6) block-sparse attention           prism_bsa_fwd / prism_bsa_bwd_*
  (7) back to THW order                prism_scatter_rows
Deliberate differences from the reference: block
means and scores are fp32 (the reference pools and scores in q's dtype) and
every reduction uses one fixed order, so zone statistics, shape ids and
selected sets are reproducible bit for bit.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import ops
from .dynamic_block_shape import ALL_CANDIDATE_SHAPES, ZONE_SIZE, _gradient_and_shapes

_TILE = 64  # kernel tile (dynamic_block_attention.py:15)


# ------------------------------------------------------------------ geometry helpers (API parity)
def _build_rearrange_index(shape_ids, ZT, ZH, ZW, H, W, device):
    """src_idx[S], inv_idx[S] int64 (dynamic_block_attention.py:107-135)."""
    return ops.rearrange_index(shape_ids.to(device), (ZT * ZONE_SIZE, H, W))


def _build_block_tile_maps(shape_ids, ZT, ZH, ZW, device):
    """(block_id_of_tile [N_tiles], kblock_tiles [N_b+1, 2], N_b, N_tiles)
    (dynamic_block_attention.py:138-170)."""
    lay = ops.ZoneLayout(shape_ids.to(device), (ZT * ZONE_SIZE, ZH * ZONE_SIZE, ZW * ZONE_SIZE))
    first = lay.block_first_tile[: lay.N_b + 1].to(torch.int64)
    two = (first[1:] - first[:-1]) == 2
    kbt = torch.full((lay.N_b + 1, 2), lay.Nt, device=device, dtype=torch.int64)
    kbt[: lay.N_b, 0] = first[:-1]
    kbt[: lay.N_b, 1] = torch.where(two, first[:-1] + 1, torch.full_like(first[:-1], lay.Nt))
    return lay.block_id_of_tile.to(torch.int64), kbt, lay.N_b, lay.Nt


# ------------------------------------------------------------------ selection (steps 3-5)
class _Plan:
    """Everything the attention kernels need for one call, built under no_grad."""

    def __init__(self, q, k, v, grid, shape_ids, valid_mask, sparsity, cdf_threshold, sm_scale,
                 compute_padded_queries=False, box=None, keep_scores=False, compact_lists=False):
        B, H, _, D = q.shape
        self.lay = ops.ZoneLayout(shape_ids, grid, box)
        lay = self.lay
        self.B, self.H, self.S, self.D = B, H, lay.S, D
        self.grid = grid
        gq = ops.gather_pool(q, lay, valid_mask, rows=True, pool=True, counts=True)
        gk = ops.gather_pool(k, lay, valid_mask, rows=True, pool=True)
        gv = ops.gather_pool(v, lay, valid_mask, rows=True)
        self.q_re, self.k_re, self.v_re = gq["rows"], gk["rows"], gv["rows"]
        # zone-grid positions outside the input grid are invalid tokens
        masked = valid_mask is not None or lay.padded
        self.kv_valid = gq["valid_re"] if masked else None
        self.block_count = gq["block_count"]
        self.tile_count = gq["tile_count"]
        scores = ops.block_scores(gq["block_mean"].view(B * H, lay.N_b, D), gk["block_mean"].view(B * H, lay.N_b, D),
                                  self.block_count if masked else None)
        sel = ops.select_tiles(scores, sparsity, cdf_threshold, sm_scale, lay.block_first_tile,
                               self.tile_count if masked else None)
        # the [B*H, N_b, N_b] scores (564 MB at 2K) are freed once the lists
        # exist, as the reference frees them per head; kept only on request
        self.scores = scores if keep_scores else None
        del scores
        self.sel = sel
        skip = masked and not compute_padded_queries
        self.qstart, self.qlen = ops.tile_rows(sel["ntiles"], lay.block_id_of_tile, B * H, lay.Nt, lay.N_b,
                                               sel["tcap"], self.tile_count if skip else None)
        self.qcols = sel["tiles"].view(-1)
        # compact lists: the two pair unions the backward keeps are stored as
        # CSR, O(nnz) memory instead of pairs x Nt (settle(); one host read of
        # both nnz, made while the forward kernel runs); same entries in the
        # same order, so identical results
        self.compact = compact_lists
        self._settled = False
        # pair unions of the per-query-tile key lists (forward, dQ) and the key
        # validity words of padded key tiles
        self.tmasks = ops.tile_masks(self.kv_valid) if masked else None
        # pair the query tiles of each zone by list overlap (fewest idle wave slots)
        self.qpair = ops.pair_tiles(self.qstart, self.qlen, self.qcols, lay.Nt)
        self.qunion = ops.pair_union(self.qstart, self.qlen, self.qcols, lay.Nt, self.tmasks, pairmap=self.qpair)
        self._csr = ops.DeferredCompaction(3) if compact_lists else None
        if compact_lists:
            self._csr.add(0, self.qunion)
        # launch order of the forward and dQ kernels (the last workgroups ids
        # take the longest lists first: the launch does not end on a long one)
        self.qorder = ops.pair_order(self.qunion[1], 64)
        # quad unions (two pairs of a zone per workgroup: four query tiles per
        # staged K / V tile), which the forward and dQ kernels walk instead of
        # the pair unions when ops.QUADS is set (same results, bit for bit)
        self.qquad = self.qquad_order = self.qquadmap = None
        # dq_quads: dQ walks them too (by default on this path), so the
        # backward keeps them
        self.quads = ops.QUADS and lay.Nt % 4 == 0
        self.dq_quads = self.quads and ops.DQ_QUADS is not False
        if self.quads:
            self.qquadmap = self.qpair
            self.qquad = ops.quad_union(self.qstart, self.qlen, self.qcols, lay.Nt, self.tmasks,
                                        pairmap=self.qquadmap)
            if compact_lists and self.dq_quads:
                self._csr.add(2, self.qquad)
            self.qquad_order = ops.pair_order(self.qquad[1], 32)
        self.klists = None
        self.kpair = None
        self.kunion = None
        self.korder = None
        self.keys_ready = None  # event of a key-list build on the side stream

    def build_key_lists_side(self):
        """build_key_lists on the side stream, after the work queued so far on
        the current stream."""
        if self.kunion is not None:
            return
        _, self.keys_ready = ops.side_launch(
            self.qcols.device, self.build_key_lists, reads=(self.qstart, self.qlen, self.qcols),
            produces=lambda _: (*self.klists, self.kpair, *self.kunion, self.korder,
                                self._csr.offsets[1] if self._csr is not None else None))

    def join_side(self):
        """Make the current stream wait for a side-stream key-list build (the
        stream fork is joined where it was opened, so a captured or
        backward-less forward leaves no dangling dependency)."""
        if self.keys_ready is not None:
            torch.cuda.current_stream().wait_event(self.keys_ready)
            self.keys_ready = None

    def build_key_lists(self):
        """Per-key-tile query lists, their pairing, unions and launch order
        (the dK/dV side), built on first use."""
        self.join_side()
        if self.kunion is not None:
            return
        Nt = self.lay.Nt
        self.klists = ops.transpose_lists(self.qstart, self.qlen, self.qcols, self.B * self.H, Nt)
        self.kpair = ops.pair_tiles(*self.klists, Nt)
        self.kunion = ops.pair_union(*self.klists, Nt, pairmap=self.kpair)
        self.korder = ops.pair_order(self.kunion[1], 32)
        if self._csr is not None:
            self._csr.add(1, self.kunion)

    def settle(self):
        """Keep only what the backward reads: the query-side and key-side pair
        unions, and the quad unions when dQ walks them (compact CSR when the
        plan is compact, with one batched host read of their nnz), pairings
        and launch orders.  The per-tile lists (1.0 GB query-side and 0.66 GB
        key-side at config 4) and the forward-only quad unions are released."""
        if self._settled:
            return
        self.build_key_lists()
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

    def list_bytes(self) -> int:
        """Bytes of the work lists the plan holds."""
        ts = [*self.qunion, self.qstart, self.qlen]
        if self.qquad is not None:
            ts += list(self.qquad)
        if self.qcols is not None:
            ts.append(self.qcols)
        if self.kunion is not None:
            ts += list(self.kunion)
        if self.klists is not None:
            ts += list(self.klists)
        return sum(t.numel() * t.element_size() for t in ts)

    def sum_lens(self) -> int:
        """Executed (query tile, key tile) pairs (host sync)."""
        return int(self.qlen.sum().item())


class _DynBSA(torch.autograd.Function):
    """Attention over a _Plan with gradients to the THW q, k, v
    (_dyn_bsa_kernel, dynamic_block_attention.py:71-101, plus the autograd of
    the gathers :250-252 and the scatter :329)."""

    @staticmethod
    def forward(ctx, q, k, v, plan: _Plan, sm_scale: float):
        grads = any(ctx.needs_input_grad[:3])
        if grads:
            # the backward's lists, beside the forward kernel (or before it)
            if ops.OVERLAP_SIDE_WORK:
                plan.build_key_lists_side()
            else:
                plan.build_key_lists()
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
        return ops.scatter_rows(o_re, plan.lay, q.dtype)

    @staticmethod
    def backward(ctx, do):
        plan: _Plan = ctx.plan
        o_re, lse = ctx.saved_tensors
        lay = plan.lay
        gd = ops.gather_pool(do.contiguous(), lay, None, rows=True, dot_with=o_re)
        do_re, delta = gd["rows"], gd["rowdot"]
        plan.build_key_lists()
        m2 = ops.lse_to_m2(lse)
        tq, tk, tv = ctx.in_dtypes
        side = {}

        def scatter_dkdv(dk_re, dv_re):
            # dK and dV back to THW order on the side stream, during the dQ kernel
            if ops.OVERLAP_SIDE_WORK and ops.OVERLAP_DKDV_SCATTER:
                side["dkdv"] = ops.side_launch(
                    dk_re.device, lambda: (ops.scatter_rows(dk_re, lay, tk), ops.scatter_rows(dv_re, lay, tv)),
                    reads=(dk_re, dv_re), produces=lambda out: out)

        quads = plan.dq_quads
        dq_re, dk_re, dv_re = ops.bsa_bwd(plan.q_re, plan.k_re, plan.v_re, do_re, m2, delta, plan.kv_valid,
                                          plan.tmasks, plan.qquad if quads else plan.qunion, plan.kunion,
                                          ctx.sm_scale, plan.qquadmap if quads else plan.qpair, plan.kpair,
                                          plan.qquad_order if quads else plan.qorder, plan.korder,
                                          after_dkdv=scatter_dkdv, q_quads=quads)
        dq = ops.scatter_rows(dq_re, lay, tq)
        if "dkdv" in side:
            (dk, dv), done = side["dkdv"]
            torch.cuda.current_stream().wait_event(done)
        else:
            dk = ops.scatter_rows(dk_re, lay, tk)
            dv = ops.scatter_rows(dv_re, lay, tv)
        return dq, dk, dv, None, None


def plan_dynamic(q, k, v, grid_padded, *, method, sparsity=0.9375, cdf_threshold=None, audio_token_norms=None,
                 valid_mask=None, lambda_a=0.5, tau_128=0.15, lambda_128=1.0, shape_ids=None,
                 compute_padded_queries=False, input_grid=None, keep_scores=False, compact_lists=False) -> _Plan:
    """Steps (1)-(5) of flash_attn_bsa_3d_dynamic: shape ids, layout, pooled
    scores, selection and tile lists (no attention).

    With input_grid (Ti, Hi, Wi) inside grid_padded, q, k, v, the audio norms
    and valid_mask cover the input grid only (S = Ti Hi Wi): the zero padding
    and padding mask of wan_video_dit.py:342-400 are applied inside the
    kernels, with results identical to padding first.  compute_padded_queries
    defaults to False here, the adapters' setting (flash_attn_bsa_3d_dynamic
    passes True unless told otherwise).  keep_scores keeps the fp32 block
    scores on the plan (plan.scores) for inspection.  compact_lists makes
    plan.settle() keep the two pair unions in compact CSR form (O(nnz)
    memory, one host read for both); the plan keeps every list until then."""
    B, Hn, S, D = q.shape
    T, H, W = grid_padded
    box = tuple(input_grid) if input_grid is not None else (T, H, W)
    assert box[0] * box[1] * box[2] == S
    assert all(0 < b <= g for b, g in zip(box, (T, H, W)))
    assert T % ZONE_SIZE == 0 and H % ZONE_SIZE == 0 and W % ZONE_SIZE == 0
    if sparsity is None and cdf_threshold is None:
        raise ValueError("Either sparsity or cdf_threshold must be provided")
    if method not in ("ivpq", "penalty") and shape_ids is None:
        raise ValueError(f"unknown dynamic-block method: {method!r}")
    sm_scale = 1.0 / (D ** 0.5)
    with torch.no_grad():
        if shape_ids is not None:
            shape_ids = torch.as_tensor(shape_ids, device=q.device)
        else:
            shape_ids = _gradient_and_shapes(v.detach(), audio_token_norms, (T, H, W), method, lambda_a, tau_128,
                                             lambda_128, valid_mask, box)[2]
        return _Plan(q.detach(), k.detach(), v.detach(), (T, H, W), shape_ids, valid_mask, sparsity, cdf_threshold,
                     sm_scale, compute_padded_queries, box, keep_scores, compact_lists)


def flash_attn_bsa_3d_dynamic(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    grid_padded: Tuple[int, int, int],
    *,
    method: str,
    sparsity: Optional[float] = 0.9375,
    cdf_threshold: Optional[float] = None,
    audio_token_norms: Optional[torch.Tensor] = None,
    valid_mask: Optional[torch.Tensor] = None,
    lambda_a: float = 0.5,
    tau_128: float = 0.15,
    lambda_128: float = 1.0,
    shape_ids: Optional[torch.Tensor] = None,
    return_shape_ids: bool = False,
    compute_padded_queries: bool = True,
    input_grid: Optional[Tuple[int, int, int]] = None,
    compact_lists: bool = True,
):
    """Dynamic-block-shape BSA for video self-attention; returns [B,H,S,D] in
    THW order (dynamic_block_attention.py:194-332).  q, k, v: [B,H,S,D] THW
    order on the GPU, grid padded to multiples of 8; float32 or bfloat16
    (attention itself runs in bf16 MFMA with fp32 accumulation).

    With a valid_mask, query tiles that hold no valid token are padding the
    caller slices away (wan_video_dit.py:429-431).  Like the reference, this
    function attends for them by default (their pooled query is 0, so the
    threshold keeps ~p of all blocks).  compute_padded_queries=False (not in
    the reference's signature; the adapters use it) gives them empty lists
    instead: their output rows are 0, and outputs at valid positions and all
    gradients of valid tokens are the same either way when the incoming
    gradient is 0 at padded positions (as the caller's unpadding makes it).

    input_grid (not in the reference's signature) takes the caller's unpadded
    grid: q, k, v [B,H,Ti*Hi*Wi,D], audio norms and valid_mask then cover it,
    grid_padded is its round-up to multiples of 8, and the output (and the
    gradients) come back unpadded.  This is the padding, valid mask and
    unpadding of wan_video_dit.py:342-431 done inside the gather and scatter
    kernels; the result equals padding first and slicing after, bit for bit.

    When gradients are needed, the forward releases the per-tile lists once
    the backward's pair unions exist.  compact_lists (not in the reference's
    signature; default True) keeps those unions in compact CSR form until
    the backward (O(nnz) memory, one host read of their sizes made while the
    forward kernel runs); False keeps them as dense pairs x Nt buffers.
    Results are identical either way."""
    plan = plan_dynamic(q, k, v, grid_padded, method=method, sparsity=sparsity, cdf_threshold=cdf_threshold,
                        audio_token_norms=audio_token_norms, valid_mask=valid_mask, lambda_a=lambda_a,
                        tau_128=tau_128, lambda_128=lambda_128, shape_ids=shape_ids,
                        compute_padded_queries=compute_padded_queries, input_grid=input_grid,
                        compact_lists=compact_lists)
    sm_scale = 1.0 / (q.shape[-1] ** 0.5)
    out = _DynBSA.apply(q, k, v, plan, sm_scale)
    if return_shape_ids:
        return out, plan.lay.shape_ids
    return out


__all__ = ["flash_attn_bsa_3d_dynamic", "plan_dynamic", "ALL_CANDIDATE_SHAPES"]
