#!/usr/bin/env bash
# The CPU test suite against AddressSanitizer + UndefinedBehaviorSanitizer builds of the CPU code:
# the oracle (oracle/_asan/liborc.so) and the C++ host program with the ingest parser
# (tests/cpp/aos_host_test_asan). Python itself is not instrumented, so the ASan runtime is
# preloaded; leak checking is off (the interpreter keeps its allocations to exit). Any sanitizer
# report aborts the process that made it and fails the test that ran it.
set -euo pipefail
ROOT="$(cd "$(dirname "$0")/.." && pwd)"
make -s -C "$ROOT/oracle" asan
make -s -C "$ROOT/tests/cpp" asan
ASAN_RT="$(gcc -print-file-name=libasan.so)"
export AOS_ORACLE_LIB="$ROOT/oracle/_asan/liborc.so"
export AOS_HOST_TEST="$ROOT/tests/cpp/aos_host_test_asan"
export ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1"
export UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1"
cd "$ROOT"
LD_PRELOAD="$ASAN_RT" python -m pytest tests -q -m "not gpu" -p no:cacheprovider "$@"
