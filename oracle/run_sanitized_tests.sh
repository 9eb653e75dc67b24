#!/bin/bash
# CPU test suite against the AddressSanitizer + UBSan build of the oracle (CPU only:
# the GPU tests are deselected). The sanitizer runtimes are preloaded because the
# interpreter itself is not instrumented; leak checking is off (the interpreter's own
# allocations at exit are not the oracle's).
set -e
ROOT="$(cd "$(dirname "$0")/.." && pwd)"
make -C "$ROOT/oracle" sanitize
ASAN="$(gcc -print-file-name=libasan.so)"
UBSAN="$(gcc -print-file-name=libubsan.so)"
export PKV_ORACLE_LIB="$ROOT/oracle/libpkv_oracle_asan.so"
export ASAN_OPTIONS="detect_leaks=0:abort_on_error=1"
export UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1"
cd "$ROOT"
LD_PRELOAD="$ASAN:$UBSAN" python -m pytest tests -q -m "not gpu" -p no:cacheprovider "$@"
