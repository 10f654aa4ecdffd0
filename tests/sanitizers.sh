#!/bin/bash
# Runs the CPU tests of the boundary (argument validation, the .gsv parser, host helpers) and of the
# oracle under AddressSanitizer + UndefinedBehaviorSanitizer: the host code of libgsvk built with
# -fsanitize=address,undefined (gpt-sovits-native_amd/_san/, device code unchanged) and the oracle
# built the same way with clang (oracle/_san/). Python itself is not instrumented, so the clang
# sanitizer runtime is preloaded; leak detection is off (the interpreter's own allocations).
# Usage: bash tests/sanitizers.sh [pytest args]   (default: the loader, ABI and oracle CPU tests)
set -euo pipefail
ROOT="$(cd "$(dirname "${BASH_SOURCE[0]}")/.." && pwd)"
make -C "$ROOT/gpt-sovits-native_amd" -j8 san >/dev/null
make -C "$ROOT/oracle" san >/dev/null
RT="$(/opt/rocm/llvm/bin/clang -print-file-name=libclang_rt.asan-x86_64.so)"
[ -f "$RT" ] || { echo "no clang ASan runtime at $RT" >&2; exit 2; }
export GSVK_LIB="$ROOT/gpt-sovits-native_amd/_san/libgsvk.so"
export GSVK_ORACLE_LIB="$ROOT/oracle/_san/liboracle.so"
export ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1"
export UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1"
if [ $# -eq 0 ]; then
  set -- "$ROOT/tests/test_gsv_loader.py" "$ROOT/tests/test_abi.py" "$ROOT/tests/test_oracle.py" \
         "$ROOT/tests/test_oracle_gemv.py" "$ROOT/tests/test_oracle_attention.py" \
         "$ROOT/tests/test_oracle_conv.py"
fi
LD_PRELOAD="$RT" python -m pytest -q -m "not gpu" -p no:cacheprovider "$@"
