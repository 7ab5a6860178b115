"""Per-zone block-shape selection, MI355X implementation.

Mirrors hymm/models/modules/block_sparse_attention/dynamic_block_shape.py of
the reference (same public names, argument meaning and errors); every
computation runs in the HIP kernels of libprism_bsa.so (prism_zone_stats,
prism_zone_gradient, prism_audio_zone_stats, prism_zone_shapes,
prism_assign_shapes).

Floating-point evaluation order is the canonical one documented in
prism_amd/csrc/stats.hip (bit-exact against the CPU oracle).  Single GPU: the
sequence-parallel AVG all-reduce of the reference (_maybe_sp_average, :132-151)
is the identity here, so ``sp_reduce`` is accepted and has no effect.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from . import ops

# dynamic_block_shape.py:6-33
CANDIDATE_SHAPES_64: List[Tuple[int, int, int]] = [
    (4, 4, 4), (8, 2, 4), (8, 4, 2), (2, 4, 8), (2, 8, 4), (4, 2, 8), (4, 8, 2),
]
CANDIDATE_SHAPES_128: List[Tuple[int, int, int]] = [
    (2, 8, 8), (8, 2, 8), (8, 8, 2), (4, 4, 8), (4, 8, 4), (8, 4, 4),
]
ALL_CANDIDATE_SHAPES: List[Tuple[int, int, int]] = CANDIDATE_SHAPES_64 + CANDIDATE_SHAPES_128
NUM_CANDIDATES_64 = len(CANDIDATE_SHAPES_64)
NUM_CANDIDATES = len(ALL_CANDIDATE_SHAPES)
ZONE_SIZE = 8
_EPS = 1e-6

_METHODS = ("ivpq", "penalty")


def candidate_tensors(device, dtype=torch.float32):
    """(shapes[C,3], log2_shapes[C,3], is_128[C], product[C]) (dynamic_block_shape.py:36-50)."""
    key = (str(device), dtype)
    cache = candidate_tensors._cache
    if key not in cache:
        shapes = torch.tensor(ALL_CANDIDATE_SHAPES, device=device, dtype=dtype)
        log2 = torch.tensor([[s.bit_length() - 1 for s in sh] for sh in ALL_CANDIDATE_SHAPES], device=device,
                            dtype=dtype)
        prod = shapes.prod(dim=-1)
        cache[key] = (shapes, log2, prod > 64.5, prod)
    return cache[key]


candidate_tensors._cache = {}


def _check_grid(grid_padded):
    T, H, W = grid_padded
    assert T % ZONE_SIZE == 0 and H % ZONE_SIZE == 0 and W % ZONE_SIZE == 0, (
        f"grid {grid_padded} must be multiple of zone size {ZONE_SIZE}")
    return int(T), int(H), int(W)


def _as_bhsd(v: torch.Tensor, grid) -> torch.Tensor:
    """[T,H,W,D] head-averaged features -> [1,1,S,D]; [B,H,S,D] passes through
    (the kernel then forms the batch-0 head mean itself)."""
    T, H, W = grid
    if v.dim() == 4 and tuple(v.shape[:3]) == (T, H, W):
        return v.reshape(1, 1, T * H * W, v.shape[-1])
    if v.dim() == 4:
        return v
    raise ValueError(f"expected [T,H,W,D] or [B,H,S,D] features, got {tuple(v.shape)}")


def compute_zone_aggregates(v_headavg_thw_d: torch.Tensor, ZT: int, ZH: int, ZW: int,
                            valid_mask_thw: Optional[torch.Tensor] = None):
    """Masked zone means (dynamic_block_shape.py:68-129).  Returns
    (packed[Nz, 25D], (t_valid, h_valid, w_valid))."""
    grid = (ZT * ZONE_SIZE, ZH * ZONE_SIZE, ZW * ZONE_SIZE)
    packed, av = ops.zone_stats(_as_bhsd(v_headavg_thw_d, grid), grid, valid_mask_thw)
    avb = av.bool()
    return packed, (avb[:, 0:8], avb[:, 8:16], avb[:, 16:24])


def compute_audio_directional(audio_norms_thw: Optional[torch.Tensor], ZT: int, ZH: int, ZW: int,
                              valid_mask_thw: Optional[torch.Tensor] = None, device=None):
    """(a_bar_norm, v_hat_T, v_hat_H, v_hat_W), each [Nz] fp32
    (dynamic_block_shape.py:189-245)."""
    Nz = ZT * ZH * ZW
    if audio_norms_thw is None:
        dev = device if device is not None else (valid_mask_thw.device if valid_mask_thw is not None else "cuda")
        z = torch.zeros(Nz, device=dev, dtype=torch.float32)
        return z, z.clone(), z.clone(), z.clone()
    grid = (ZT * ZONE_SIZE, ZH * ZONE_SIZE, ZW * ZONE_SIZE)
    abar, vhat = ops.audio_zone_stats(audio_norms_thw.reshape(-1), grid, valid_mask_thw)
    a_norm = abar / abar.max().clamp(min=_EPS)
    return a_norm, vhat[:, 0].contiguous(), vhat[:, 1].contiguous(), vhat[:, 2].contiguous()


def _gradient_and_shapes(v, audio_norms_thw, grid, method, lambda_a, tau_128, lambda_128, valid_mask_thw, box=None):
    """Shape ids of the zone grid `grid`; v, the audio norms and the mask cover
    the input grid `box` inside it (default: grid itself)."""
    if method not in _METHODS:
        raise ValueError(f"unknown dynamic-block method: {method!r}")
    D = v.shape[-1]
    packed, av = ops.zone_stats(v, grid, valid_mask_thw, box)
    rho_raw, aniso = ops.zone_gradient(packed, av, D)
    abar = vhat = None
    if audio_norms_thw is not None:
        abar, vhat = ops.audio_zone_stats(audio_norms_thw.reshape(-1), grid, valid_mask_thw, box)
    return ops.zone_shapes(rho_raw, aniso, abar, vhat, method, lambda_a, tau_128, lambda_128)


def compute_effective_gradient(v_headavg_thw_d: torch.Tensor, audio_norms_thw: Optional[torch.Tensor],
                               ZT: int, ZH: int, ZW: int, lambda_a: float = 0.5,
                               valid_mask_thw: Optional[torch.Tensor] = None, sp_reduce: bool = True):
    """(g[Nz,3], rho[Nz]) (dynamic_block_shape.py:248-301)."""
    grid = (ZT * ZONE_SIZE, ZH * ZONE_SIZE, ZW * ZONE_SIZE)
    g, rho, _ = _gradient_and_shapes(_as_bhsd(v_headavg_thw_d, grid), audio_norms_thw, grid, "ivpq",
                                     lambda_a, 0.15, 1.0, valid_mask_thw)
    return g, rho


def _assign(g: torch.Tensor, rho: torch.Tensor, method: int, tau_128: float, lambda_128: float) -> torch.Tensor:
    return ops.assign_shapes(g, rho, method, tau_128, lambda_128)


def select_shapes_ivpq(g: torch.Tensor, rho: torch.Tensor, tau_128: float = 0.15) -> torch.Tensor:
    """IVPQ nearest candidate in log2 space (dynamic_block_shape.py:303-327)."""
    return _assign(g, rho, 0, tau_128, 1.0)


def select_shapes_penalty(g: torch.Tensor, rho: torch.Tensor, tau_128: float = 0.15,
                          lambda_128: float = 1.0) -> torch.Tensor:
    """Penalty matching (dynamic_block_shape.py:330-355)."""
    return _assign(g, rho, 1, tau_128, lambda_128)


def select_zone_shapes(v_headavg_thw_d: torch.Tensor, audio_norms_thw: Optional[torch.Tensor],
                       grid_padded: Tuple[int, int, int], method: str, lambda_a: float = 0.5,
                       tau_128: float = 0.15, lambda_128: float = 1.0,
                       valid_mask_thw: Optional[torch.Tensor] = None, sp_reduce: bool = True) -> torch.Tensor:
    """Features -> shape id per zone, int64 [Nz] (dynamic_block_shape.py:358-391).

    ``v_headavg_thw_d`` is the head-averaged [T,H,W,D] tensor of the reference,
    or the full V [B,H,S,D]: the kernel then fuses the batch-0 head mean
    (dynamic_block_attention.py:236) into its single pass over V.
    """
    grid = _check_grid(grid_padded)
    return _gradient_and_shapes(_as_bhsd(v_headavg_thw_d, grid), audio_norms_thw, grid, method, lambda_a,
                                tau_128, lambda_128, valid_mask_thw)[2]


__all__ = [
    "CANDIDATE_SHAPES_64", "CANDIDATE_SHAPES_128", "ALL_CANDIDATE_SHAPES", "NUM_CANDIDATES_64", "NUM_CANDIDATES",
    "ZONE_SIZE", "candidate_tensors", "compute_zone_aggregates", "compute_audio_directional",
    "compute_effective_gradient", "select_shapes_ivpq", "select_shapes_penalty", "select_zone_shapes",
]
