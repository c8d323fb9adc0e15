#!/bin/bash
# Runs the CPU test suite against AddressSanitizer + UBSan builds of the C host layer
# (platform, registry, operators' host code, graph, fusion pass, session) and of the
# oracle.  CPU only: the HIP device code is not instrumented and no GPU is used.
#   tests/sanitize.sh [extra pytest args]
set -euo pipefail
ROOT="$(cd "$(dirname "$0")/.." && pwd)"
make -C "$ROOT/cudaforge_amd/csrc" -j8 sanitize
make -C "$ROOT/oracle" sanitize
ASAN_LIB="$(gcc -print-file-name=libasan.so)"
UBSAN_LIB="$(gcc -print-file-name=libubsan.so)"
cd "$ROOT"
LD_PRELOAD="$ASAN_LIB:$UBSAN_LIB" \
ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:strict_string_checks=1:detect_stack_use_after_return=1" \
UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1" \
CUDAFORGE_AMD_LIB="$ROOT/cudaforge_amd/csrc/_build_san/libcudaforge_amd.so" \
CUDAFORGE_ORACLE_SO="$ROOT/oracle/_build_san/liboracle.so" \
    python -m pytest "$ROOT/tests" -m "not gpu" -q -p no:cacheprovider "$@"
echo "sanitized libraries: $ROOT/cudaforge_amd/csrc/_build_san/libcudaforge_amd.so, $ROOT/oracle/_build_san/liboracle.so"
