#!/bin/bash
# CPU test runs under AddressSanitizer + UndefinedBehaviorSanitizer (no GPU).
#  1. the CPU oracle (oracle/bsa_oracle.c, gcc) instrumented, the whole
#     CPU test suite on it, under gcc's ASan runtime;
#  2. the host code of libprism_bsa.so (argument checks, list checks;
#     hipcc -Xarch_host) instrumented, the C-ABI tests on it, under clang's
#     ASan runtime.
# Any report aborts the run (halt_on_error, -fno-sanitize-recover=all).
set -euo pipefail
ROOT="$(cd "$(dirname "$0")/.." && pwd)"
cd "$ROOT"
export ASAN_OPTIONS=detect_leaks=0:halt_on_error=1:abort_on_error=1
export UBSAN_OPTIONS=halt_on_error=1:print_stacktrace=1
STDCXX="$(gcc -print-file-name=libstdc++.so.6)"  # preloaded too: ASan must see its __cxa_throw

make -s -C oracle liboracle_san.so
echo "[sanitizers] CPU suite on the ASan/UBSan oracle"
LD_PRELOAD="$(gcc -print-file-name=libasan.so) $STDCXX" PRISM_ORACLE_LIB="$ROOT/oracle/liboracle_san.so" \
    python -m pytest tests/ -x -q -m "not gpu" -p no:cacheprovider

python prism_amd/build.py --sanitize
ASANRT="$(ls /opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so | head -1)"
echo "[sanitizers] C-ABI tests on the host-sanitized library"
LD_PRELOAD="$ASANRT $STDCXX" PRISM_BSA_LIB="$ROOT/prism_amd/_build_san/libprism_bsa_san.so" \
    python -m pytest tests/test_capi.py tests/test_list_checks.py -x -q -p no:cacheprovider
echo "[sanitizers] clean"
