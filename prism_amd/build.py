"""Build libprism_bsa.so (HIP, gfx950) in-tree.

    python prism_amd/build.py          # run as a file: importing the package
                                       # would load the library it builds
    PRISM_DEBUG=1 python prism_amd/build.py   # debug build: work lists checked
                                              # on the host before every launch
    python prism_amd/build.py --sanitize      # host code under ASan + UBSan
                                              # (_build_san/, CPU test runs only)

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
           "oproj.hip", "validate.hip", "peak.hip"]
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


# AddressSanitizer + UBSan on the host code only (device code is built as
# usual): the argument checks and host-side list checks of the C-ABI, run on
# the CPU under clang's ASan runtime (tests/run_sanitizers.sh)
SANITIZE_DIR = os.path.join(HERE, "_build_san")
SANITIZE_LIB = os.path.join(SANITIZE_DIR, "libprism_bsa_san.so")
HOST_SANITIZE_FLAGS = ["-g", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                       "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer"]


def _compile(src: str, sanitize: bool = False) -> str:
    obj = os.path.join(SANITIZE_DIR if sanitize else BUILD_DIR, os.path.splitext(src)[0] + ".o")
    flags = list(COMMON_FLAGS) + (HOST_SANITIZE_FLAGS if sanitize else [])
    if src in CANONICAL:
        flags.append("-ffp-contract=off")
    if src == "validate.hip" and os.environ.get("PRISM_DEBUG", "0") not in ("", "0"):
        # debug build: the attention entry points check their work lists on
        # the host before every launch unless PRISM_DEBUG=0 at run time
        flags.append("-DPRISM_DEBUG_DEFAULT=1")
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


def build_sanitized(verbose: bool = False) -> str:
    """The host-sanitized variant of libprism_bsa.so (_build_san/, never
    loaded unless PRISM_BSA_LIB names it; not shipped)."""
    os.makedirs(SANITIZE_DIR, exist_ok=True)
    jobs = min(len(SOURCES), max(1, int(os.environ.get("MAX_JOBS", "8"))))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, sanitize=True), SOURCES))
    cmd = [_hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-Xarch_host", "-fsanitize=address", "-Xarch_host",
           "-fsanitize=undefined", "-Xarch_host", "-shared-libsan", *objs, "-o", SANITIZE_LIB]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"sanitized link failed:\n{r.stderr[-4000:]}")
    if verbose:
        print(f"built {SANITIZE_LIB}")
    return SANITIZE_LIB


if __name__ == "__main__":
    if "--sanitize" in sys.argv[1:]:
        build_sanitized(verbose=True)
    else:
        build(verbose=True)
    sys.exit(0)
