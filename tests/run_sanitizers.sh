#!/bin/bash
# CPU runs under AddressSanitizer + UndefinedBehaviorSanitizer (no GPU needed):
#  1. the oracle (oracle/_asan/liboracle.so, gcc) under every CPU test that
#     calls it;
#  2. the library's host code (janus_amd/_build_san/libjanus_hip_san.so, hipcc
#     with the sanitizers on the host compilation only) under the C-ABI
#     validation tests.
# Python itself is not instrumented, so the sanitizer runtimes are preloaded and
# leak detection (which would report the interpreter's own allocations) is off.
set -euo pipefail
ROOT="$(cd "$(dirname "$0")/.." && pwd)"
cd "$ROOT"
make -s -C oracle asan
python -m janus_amd.build --sanitize
export ASAN_OPTIONS=detect_leaks=0:abort_on_error=1
export UBSAN_OPTIONS=print_stacktrace=1:halt_on_error=1
GCC_ASAN="$(gcc -print-file-name=libasan.so)"
GCC_UBSAN="$(gcc -print-file-name=libubsan.so)"
echo "== oracle (gcc ASan + UBSan)"
LD_PRELOAD="$GCC_ASAN:$GCC_UBSAN" JANUS_ORACLE_LIB="$ROOT/oracle/_asan/liboracle.so" \
    python -m pytest tests -q -m "not gpu" -p no:cacheprovider
CLANG_ASAN="$(/opt/rocm/llvm/bin/clang -print-resource-dir)/lib/linux/libclang_rt.asan-x86_64.so"
echo "== host library (clang ASan + UBSan)"
LD_PRELOAD="$CLANG_ASAN" JANUS_LIB="$ROOT/janus_amd/_build_san/libjanus_hip_san.so" \
    python -m pytest tests/test_abi.py -q -m "not gpu" -p no:cacheprovider
