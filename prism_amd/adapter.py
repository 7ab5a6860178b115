"""Caller-side adapter: the contract of SelfAttention._run_bsa_dynamic
(hymm/models/modules/wan_video_dit.py:342-432) and the A2V norm computation
(wan_video_dit.py:739-752), on top of flash_attn_bsa_3d_dynamic; and the plain
uniform-shape branch of SelfAttention._run_bsa (run_bsa_uniform).

The reference pads T, H, W up to multiples of ZONE_SIZE, builds the valid
mask of the padded grid, pads the audio norms with zeros, and unpads the
output.  Here the kernels read the unpadded tensors directly (grid positions
outside the input are zero, invalid tokens), so none of those copies is made;
outputs and gradients equal the pad + call + slice flow bit for bit.  Cached
shape ids are reused within one training forward pass (activation-checkpoint
recompute).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import ops
from .dynamic_block_attention import flash_attn_bsa_3d_dynamic
from .dynamic_block_shape import ZONE_SIZE
from .uniform_block_attention import bsa_chunked

# default bsa_params keys and values read by the reference (wan_video_dit.py:415-421)
DEFAULT_BSA_PARAMS = {
    "sparsity": 0.9375,
    "cdf_threshold": None,
    "dynamic_block_lambda_a": 0.5,
    "dynamic_block_tau_128": 0.15,
    "dynamic_block_lambda_128": 1.0,
}


def a2v_token_norms(a2v_bridge_residual: torch.Tensor) -> torch.Tensor:
    """||residual[0, m, :]||_2 per token, in the residual's dtype
    (wan_video_dit.py:742-752, single GPU: no all-gather)."""
    with torch.no_grad():
        return ops.a2v_norms(a2v_bridge_residual)


def a2v_bridge_projection(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None):
    """The a2v bridge's output projection with the residual norms fused:
    residual = x weight^T + bias (ConditionalCrossAttention.o,
    hymm/models/modules/interactionv2.py:225, :348; the a2v_bridge_residual of
    mova.py:127-137) and ||residual[0, m, :]||_2 (wan_video_dit.py:742-752)
    formed in the projection's epilogue instead of a second read of the
    residual.  x: [B, S, K] or [S, K] bf16; weight: [C, K] bf16; bias: [C]
    bf16 or None (C a multiple of 256, K of 64).  Returns (residual in x's
    layout with C channels, norms [S] bf16 of batch 0)."""
    lead = x.shape[:-1]
    y, norms = ops.linear_rownorm(x.reshape(-1, x.shape[-1]), weight, bias)
    S = x.shape[-2] if x.dim() == 3 else x.shape[0]
    return y.view(*lead, weight.shape[0]), norms[:S]


def padded_grid(grid_size):
    T, H, W = grid_size
    pt = (ZONE_SIZE - T % ZONE_SIZE) % ZONE_SIZE
    ph = (ZONE_SIZE - H % ZONE_SIZE) % ZONE_SIZE
    pw = (ZONE_SIZE - W % ZONE_SIZE) % ZONE_SIZE
    return (T + pt, H + ph, W + pw), (pt, ph, pw)


def valid_mask_for(grid_size, device) -> Optional[torch.Tensor]:
    """Bool [S_p] mask of real tokens in the padded grid (None if no padding)."""
    T, H, W = grid_size
    (Tp, Hp, Wp), pads = padded_grid(grid_size)
    if not any(pads):
        return None
    it = torch.arange(Tp, device=device)
    ih = torch.arange(Hp, device=device)
    iw = torch.arange(Wp, device=device)
    return ((it[:, None, None] < T) & (ih[None, :, None] < H) & (iw[None, None, :] < W)).reshape(-1).contiguous()


class DynamicBlockSparseAttention:
    """State the reference keeps on SelfAttention for the dynamic path: the
    bsa_params dict, the method switch and the per-pass shape cache
    (wan_video_dit.py:22-33, :401-427).  One key beyond the reference's:
    bsa_params["compact_lists"] (default True) keeps the work lists in
    compact CSR form until the backward (O(nnz) memory; identical results;
    False: dense buffers)."""

    def __init__(self, method: str = "ivpq", bsa_params: Optional[dict] = None):
        if method not in ("ivpq", "penalty"):
            raise ValueError(f"unknown dynamic-block method: {method!r}")
        self.method = method
        self.bsa_params = dict(DEFAULT_BSA_PARAMS)
        if bsa_params:
            self.bsa_params.update(bsa_params)
        self.training = False
        self.pass_id = 0
        self._dyn_shape_cache = None

    def advance_pass(self) -> int:
        """Call once per real outer forward (advance_dynamic_block_pass_id)."""
        self.pass_id += 1
        return self.pass_id

    def __call__(self, q_bhsd, k_bhsd, v_bhsd, grid_size, audio_token_norms=None):
        return self.run_bsa_dynamic(q_bhsd, k_bhsd, v_bhsd, grid_size, audio_token_norms)

    def run_bsa_dynamic(self, q_bhsd, k_bhsd, v_bhsd, grid_size, audio_token_norms=None):
        T, H, W = grid_size
        B, n_heads, S, D = q_bhsd.shape
        if S != T * H * W:
            raise ValueError(f"sequence length {S} != T*H*W of grid {tuple(grid_size)}")
        (Tp, Hp, Wp), _ = padded_grid(grid_size)
        grid_padded = (Tp, Hp, Wp)
        cached = None
        if self.training and self._dyn_shape_cache is not None:
            pid, g, ids = self._dyn_shape_cache
            if pid == self.pass_id and g == grid_padded:
                cached = ids
        p = self.bsa_params
        out, used = flash_attn_bsa_3d_dynamic(
            q_bhsd, k_bhsd, v_bhsd, grid_padded, method=self.method,
            sparsity=p.get("sparsity", 0.9375), cdf_threshold=p.get("cdf_threshold", None),
            audio_token_norms=None if audio_token_norms is None else audio_token_norms.reshape(-1),
            lambda_a=p.get("dynamic_block_lambda_a", 0.5), tau_128=p.get("dynamic_block_tau_128", 0.15),
            lambda_128=p.get("dynamic_block_lambda_128", 1.0), shape_ids=cached, return_shape_ids=True,
            input_grid=(T, H, W), compute_padded_queries=False,  # padded rows are sliced away (:429-431)
            compact_lists=bool(p.get("compact_lists", True)))
        if self.training:
            self._dyn_shape_cache = (self.pass_id, grid_padded, used)
        return out


# bsa_params keys the uniform branch does not pass to the kernel (wan_video_dit.py:511-520)
GUIDANCE_ONLY_KEYS = ("audio_boost_gamma", "audio_weighted_lambda", "timestep_gate_mode", "timestep_gate_power",
                      "timestep_gate_scale", "timestep_gate_threshold", "variance_boost_gamma", "taylor_alpha_f",
                      "dynamic_block_lambda_a", "dynamic_block_tau_128", "dynamic_block_lambda_128")


def run_bsa_uniform(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, grid_size, bsa_params: dict,
                    compute_padded_queries: bool = False) -> torch.Tensor:
    """The plain uniform-shape branch of SelfAttention._run_bsa
    (wan_video_dit.py:470-507 padding, :674-686 flash_attn_bsa_3d, :688-692
    unpadding): T, H, W are padded up to multiples of the per-axis maximum of
    chunk_3d_shape_q / _k (default 4x4x4), the padding is masked, and the
    output has the unpadded THW shape.  Here the padding, the rearrangement
    and the unpadding happen inside the chunk gather / scatter kernels (no
    padded copies of q, k, v or the output).  bsa_params["compact_lists"]
    keeps the work lists in compact CSR form, as in the dynamic branch."""
    B, Hn, S, D = q.shape
    T, H, W = (int(x) for x in grid_size)
    assert T * H * W == S
    kw = {key: val for key, val in bsa_params.items() if key not in GUIDANCE_ONLY_KEYS}
    cq = tuple(kw.get("chunk_3d_shape_q", (4, 4, 4)))
    ck = tuple(kw.get("chunk_3d_shape_k", (4, 4, 4)))
    ct, ch, cw = max(cq[0], ck[0]), max(cq[1], ck[1]), max(cq[2], ck[2])
    pgrid = (-(-T // ct) * ct, -(-H // ch) * ch, -(-W // cw) * cw)
    lq = ops.ChunkLayout((T, H, W), cq, q.device, pgrid=pgrid)
    lk = ops.ChunkLayout((T, H, W), ck, q.device, pgrid=pgrid)
    return bsa_chunked(q, k, v, lq, lk, sparsity=kw.get("sparsity", 0.875), cdf_threshold=kw.get("cdf_threshold"),
                       sm_scale=1.0 / (D ** 0.5), compute_padded_queries=compute_padded_queries,
                       compact_lists=bool(kw.get("compact_lists", True)))

