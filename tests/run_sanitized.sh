#!/bin/bash
# The CPU test suite with the oracle (oracle/_build_san) and the library's
# host code (qwen-omni-inference-rs_amd/lq8/liblq8_san.so) built under
# AddressSanitizer + UndefinedBehaviorSanitizer.  The interpreter itself is
# not instrumented, so clang's sanitizer runtime is preloaded; leak checks are
# off (the interpreter's own allocations would swamp them).
#   tests/run_sanitized.sh [pytest args]
set -euo pipefail
ROOT="$(cd "$(dirname "$0")/.." && pwd)"
make -C "$ROOT/oracle" sanitize
make -C "$ROOT/qwen-omni-inference-rs_amd" -j8 sanitize
RT="$(/opt/rocm/llvm/bin/clang -print-resource-dir)/lib/linux/libclang_rt.asan-x86_64.so"
export LD_PRELOAD="$RT"
export ASAN_OPTIONS=detect_leaks=0:abort_on_error=1
export UBSAN_OPTIONS=print_stacktrace=1:halt_on_error=1
export LQ8_LIBRARY="$ROOT/qwen-omni-inference-rs_amd/lq8/liblq8_san.so"
export LQ8_ORACLE_BUILD="$ROOT/oracle/_build_san"
cd "$ROOT"
exec python -m pytest tests -q -m "not gpu" -p no:cacheprovider "$@"
