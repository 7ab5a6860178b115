"""prism_amd: MI355X-native (gfx950) block-sparse attention path of
Tencent-Hunyuan/Prism, behind the reference's module API.

Public surface (reference names):
  flash_attn_bsa_3d_dynamic   dynamic_block_attention.py:194
  select_zone_shapes          dynamic_block_shape.py:358
  DynamicBlockSparseAttention SelfAttention._run_bsa_dynamic contract
  flash_attn_bsa_3d           bsa_interface.py:1123 (uniform chunk shapes)
  flash_attn_bsa_cross        bsa_interface.py:1276 (3-D / 1-D cross-modal)
  flash_attn_bsa              bsa_interface.py:683 (_attention_bsa.apply)
  a2v_token_norms             wan_video_dit.py:742-752 (A2V residual norms)
  a2v_bridge_projection       interactionv2.py:348 o-projection with the norms fused
All compute runs in libprism_bsa.so, reached through the torch.ops.prism
operators of libprism_torch.so (build: python prism_amd/build.py).
"""
from .dynamic_block_shape import (  # noqa: F401
    ALL_CANDIDATE_SHAPES, CANDIDATE_SHAPES_64, CANDIDATE_SHAPES_128, NUM_CANDIDATES, NUM_CANDIDATES_64, ZONE_SIZE,
    compute_audio_directional, compute_effective_gradient, compute_zone_aggregates, select_shapes_ivpq,
    select_shapes_penalty, select_zone_shapes,
)
from .dynamic_block_attention import _TILE, flash_attn_bsa_3d_dynamic, plan_dynamic  # noqa: F401
from .adapter import DynamicBlockSparseAttention, a2v_bridge_projection, a2v_token_norms, valid_mask_for  # noqa: F401
from .uniform_block_attention import flash_attn_bsa, flash_attn_bsa_3d, flash_attn_bsa_cross  # noqa: F401

__version__ = "0.1.0"
