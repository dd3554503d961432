#!/bin/bash
# Host-code sanitizers (no GPU): build the library with AddressSanitizer and
# UndefinedBehaviorSanitizer in its host pass (mask_amd.build --sanitize) and
# run the CPU tests that drive its host code -- the CSR -> SR-BCRS converter,
# the packings and row orders (threaded), the schedule builders, the export
# and error paths -- against it.  Any sanitizer report aborts the run.
# Usage: bash tests/sanitize_host.sh   (from the repository root)
set -euo pipefail
cd "$(dirname "$0")/.."
LIB=$(python -m mask_amd.build --sanitize | tail -1)
ASAN_RT=$(/opt/rocm/llvm/bin/clang -print-file-name=libclang_rt.asan-x86_64.so)
export MASK_AMD_SRBCRS_LIB="$LIB"
export ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1"
export UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1"
LD_PRELOAD="$ASAN_RT" python -m pytest -q -m "not gpu" -p no:cacheprovider \
  tests/test_host.py tests/test_property.py tests/test_golden.py tests/test_mtx.py "$@"
