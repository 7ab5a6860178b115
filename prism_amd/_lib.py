"""ctypes binding of libprism_bsa.so (the C-ABI of include/prism_bsa.h).

The library is the only compute path: if it is missing or a call fails the
error propagates (there is no CPU or PyTorch fallback).
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libprism_bsa.so")

P = ctypes.c_void_p
I32 = ctypes.c_int
I64 = ctypes.c_int64
F32 = ctypes.c_float
U64 = ctypes.c_uint64

# name -> argtypes (every function returns int; the last argument is the stream)
SIGNATURES = {
    "prism_zone_stats": [P, I32, I32, I64, I32, P, I32, I32, I32, I32, I32, I32, P, P, P],
    "prism_audio_zone_stats": [P, I32, P, I32, I32, I32, I32, I32, I32, P, P, P],
    "prism_zone_gradient": [P, P, I32, I32, P, P, P],
    "prism_zone_shapes": [P, P, P, P, I32, I32, F32, F32, F32, P, P, P, P],
    "prism_assign_shapes": [P, P, I32, I32, F32, F32, P, P],
    "prism_a2v_norms": [P, I32, I64, I32, P, I32, P],
    "prism_linear_rownorm": [P, P, P, I64, I32, I32, P, P, I32, P, P],
    "prism_zone_layout": [P, I32, P, P, P, P],
    "prism_rearrange_index": [P, I32, I32, I32, P, P, P],
    "prism_gather_pool": [P, I32, I32, I32, I64, I32, P, P, P, I32, I32, I32, I32, I32, I32, I64, P, P, P, P, P, P, P, P],
    "prism_scatter_rows": [P, I32, I32, I64, I32, P, I32, I32, I32, I32, I32, I32, P, I32, P],
    "prism_chunk_gather_pool": [P, I32, I32, I32, I32, P, I32, I32, I32, I32, I32, I32, I32, I32, I32, I64,
                                P, P, P, P, P, P, P, P],
    "prism_chunk_scatter_rows": [P, I32, I32, I32, I32, I32, I32, I32, I32, I32, I32, I32, I32, I64, P, I32, P],
    "prism_block_scores": [P, P, P, I32, I64, I64, I32, P, P],
    "prism_select_tiles": [P, I64, I64, I32, I64, I64, F32, U64, P, P, I64, P, P, P, I64, P, P],
    "prism_tile_rows": [P, P, P, I32, I64, I64, I64, P, P, P],
    "prism_transpose_lists": [P, P, P, I32, I64, I64, P, I64, P, P, P, P],
    "prism_transpose_lists_noalloc": [P, P, P, I32, I64, I64, I64, P, P, P, P],
    "prism_pair_union": [P, P, P, I64, I64, I64, P, P, I64, P, P, P, P],
    "prism_quad_union": [P, P, P, I64, I64, I64, P, P, I64, P, P, P, P],
    "prism_pair_tiles": [P, P, P, I64, I64, I64, P, P],
    "prism_pair_order": [P, I64, I32, I64, P, P],
    "prism_lists_csr_offsets": [P, I64, P, P, P],
    "prism_lists_csr_fill": [P, P, P, I64, P, P, P],
    "prism_tile_masks": [P, I64, P, P],
    "prism_lse_to_m2": [P, I64, P, P],
    "prism_bsa_fwd": [P, P, P, I32, I64, I64, I32, P, P, P, P, P, P, F32, P, P, P, P],
    "prism_bsa_fwd_quad": [P, P, P, I32, I64, I64, I32, P, P, P, P, P, P, F32, P, P, P, P],
    "prism_bwd_preprocess": [P, P, I64, I32, P, P],
    "prism_bsa_bwd_dkdv": [P, P, P, P, P, P, I32, I64, I64, I32, P, P, P, P, P, P, F32, P, P, P, P],
    "prism_bsa_bwd_dq": [P, P, P, P, P, P, I32, I64, I64, I32, P, P, P, P, P, P, F32, P, P, P],
    "prism_bsa_bwd_dq_quad": [P, P, P, P, P, P, I32, I64, I64, I32, P, P, P, P, P, P, F32, P, P, P],
    "prism_check_lists": [P, P, P, I64, I64, I64, I32, P],
    "prism_mfma_peak": [I64, P, I64, P, P, P],
    "prism_copy_peak": [P, P, I64, P],
    "prism_tile_stream_peak": [P, I64, I64, P, I64, P, P],
    "prism_check_launch_maps": [P, I64, I64, P, I64],
}

_lib = None
_lock = threading.Lock()


class PrismError(RuntimeError):
    """A prism_bsa C-ABI call failed (message from prism_last_error)."""


def load() -> ctypes.CDLL:
    """Load libprism_bsa.so (built by prism_amd.build); raise if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        # PRISM_BSA_LIB: another build of the same sources (the host-sanitized
        # variant of build.py --sanitize, for CPU test runs)
        path = os.environ.get("PRISM_BSA_LIB") or LIB_PATH
        if not os.path.exists(path):
            raise ImportError(
                f"{path} not found: build the HIP library first (python prism_amd/build.py); "
                "prism_amd has no fallback path")
        lib = ctypes.CDLL(path)
        lib.prism_last_error.restype = ctypes.c_char_p
        lib.prism_last_error.argtypes = []
        lib.prism_abi_version.restype = ctypes.c_int
        lib.prism_abi_version.argtypes = []
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = args
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Call a C-ABI entry point; raise ValueError / PrismError on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.prism_last_error().decode(errors="replace")
        if rc == 1:
            raise ValueError(msg)
        raise PrismError(msg)
