#!/bin/bash
# The CPU suite (pytest -m "not gpu") against ASan + UBSan builds of the host
# library (libf3s_host.so: loader, binary graph files, generators, window
# order) and of the oracle.  CPU only; run from the repository root:
#   bash tests/sanitize.sh
# Any sanitizer report ends the run with a non-zero status.
set -euo pipefail
cd "$(dirname "$0")/.."
python3 -m fused3s_amd.build --sanitize -q
export F3S_LIB_DIR="$PWD/fused3s_amd/_build/san"
export F3S_ORACLE_LIB="$PWD/oracle/_san/liboracle.so"
# Python itself is not instrumented: leaks of the interpreter are not ours.
# Reports go to files (pytest captures the terminal of an aborted process).
logs="$(mktemp -d)"
export ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:allocator_may_return_null=1:log_path=$logs/asan"
export UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1:log_path=$logs/ubsan"
rc=0
LD_PRELOAD="$(gcc -print-file-name=libasan.so) $(gcc -print-file-name=libubsan.so)" \
    python3 -m pytest tests -m "not gpu" -x -q -p no:cacheprovider "$@" || rc=$?
if compgen -G "$logs/*" > /dev/null; then
    echo "sanitizer reports:"
    cat "$logs"/*
    rc=1
fi
rm -rf "$logs"
exit $rc
