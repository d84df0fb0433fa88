#!/usr/bin/env bash
# The CPU test suite (-m "not gpu") against AddressSanitizer +
# UndefinedBehaviorSanitizer builds of the oracle (oracle/_build/asan/) and of
# the C-ABI library's host code (phantom_moe/lib/asan/).  Both are built with
# the ROCm LLVM toolchain so they share one sanitizer runtime, which is
# preloaded into the (uninstrumented) Python interpreter.  No GPU is needed.
#
#   bash tests/run_sanitized.sh [extra pytest arguments]
set -euo pipefail
ROOT="$(cd "$(dirname "${BASH_SOURCE[0]}")/.." && pwd)"
CLANG=${CLANG:-/opt/rocm/llvm/bin/clang}
make -s -C "$ROOT/oracle" asan
(cd "$ROOT/solution-is-all-you-need_amd" && python -m phantom_moe._build --sanitize > /dev/null)
RT="$("$CLANG" -print-file-name=libclang_rt.asan-x86_64.so)"
export LD_PRELOAD="$RT"
export LD_LIBRARY_PATH="$(dirname "$RT")${LD_LIBRARY_PATH:+:$LD_LIBRARY_PATH}"
# The interpreter and torch keep memory until exit: leak reports would be noise.
export ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:symbolize=1"
export UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1"
export PHANTOM_ORACLE_LIB="$ROOT/oracle/_build/asan/libmoe_oracle.so"
export PHANTOM_MOE_LIB="$ROOT/solution-is-all-you-need_amd/phantom_moe/lib/asan/libphantom_moe.so"
cd "$ROOT"
exec python -m pytest tests -m "not gpu" -q -p no:cacheprovider "$@"
