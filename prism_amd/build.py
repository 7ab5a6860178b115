"""Build libprism_bsa.so (HIP, gfx950) in-tree.

    python prism_amd/build.py          # run as a file: importing the package
                                       # would load the library it builds

Each csrc/*.hip file is compiled by hipcc for gfx950 only and linked into one
shared library exporting the C-ABI declared in include/prism_bsa.h;
csrc/torch_ops.cpp (host C++, no device code) is built on top of it into
libprism_torch.so, the TORCH_LIBRARY(prism) operators.  Files
whose results are bit-exact parity targets are compiled with
-ffp-contract=off (their fused operations are written out explicitly).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_NAME = "libprism_bsa.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
TORCH_OPS_SRC = "torch_ops.cpp"
TORCH_OPS_PATH = os.path.join(HERE, "libprism_torch.so")

SOURCES = ["errors.hip", "stats.hip", "layout.hip", "select.hip", "lists.hip", "attn_fwd.hip", "attn_bwd.hip",
           "oproj.hip"]
CANONICAL = {"stats.hip", "layout.hip", "select.hip"}

COMMON_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # packed fp32 vector ops stay disabled on this fleet
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the prism_bsa HIP library cannot be built")


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    flags = list(COMMON_FLAGS)
    if src in CANONICAL:
        flags.append("-ffp-contract=off")
    cmd = [_hipcc(), *flags, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-4000:]}")
    return obj


def _torch_ops_cmd(out: str):
    """g++ line of the PyTorch operator library (csrc/torch_ops.cpp): torch's
    headers and libraries, HIP's runtime headers, linked against
    libprism_bsa.so found next to it at load time."""
    import torch
    from torch.utils import cpp_extension
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    inc = [f"-I{d}" for d in cpp_extension.include_paths()] + [f"-I{os.path.join(rocm, 'include')}"]
    libs = [f"-L{d}" for d in cpp_extension.library_paths()]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return [os.environ.get("CXX", "g++"), "-std=c++17", "-O2", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__=1",
            f"-D_GLIBCXX_USE_CXX11_ABI={abi}", *inc, os.path.join(CSRC, TORCH_OPS_SRC), "-o", out, *libs,
            f"-L{HERE}", "-lprism_bsa", "-ltorch", "-ltorch_cpu", "-lc10", "-lc10_hip", "-Wl,-rpath,$ORIGIN"]


def build_torch_ops(verbose: bool = False) -> str:
    """Compile libprism_torch.so, the TORCH_LIBRARY(prism) registration of
    the C-ABI (needs libprism_bsa.so built first)."""
    tmp = TORCH_OPS_PATH + ".tmp"
    r = subprocess.run(_torch_ops_cmd(tmp), capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"torch operator library failed to build:\n{r.stderr[-4000:]}")
    os.replace(tmp, TORCH_OPS_PATH)
    if verbose:
        print(f"built {TORCH_OPS_PATH}")
    return TORCH_OPS_PATH


def build(verbose: bool = False) -> str:
    """Compile every HIP source for gfx950, link libprism_bsa.so, and build
    the PyTorch operator library on top of it (the two builds overlap)."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    jobs = min(len(SOURCES), max(1, int(os.environ.get("MAX_JOBS", "8"))))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    build_torch_ops(verbose)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
