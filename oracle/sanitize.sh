#!/bin/sh
# CPU-only check of the oracle (the parity checker) under AddressSanitizer and
# UndefinedBehaviorSanitizer: builds gs_oracle.c with both (plus the
# float-to-int overflow check, which -fsanitize=undefined leaves out in gcc)
# into oracle/_san/, then runs the oracle's CPU tests against that build.
# Any report aborts the run.  Extra arguments go to pytest.
set -e
here=$(cd "$(dirname "$0")" && pwd)
out="$here/_san"
mkdir -p "$out"
gcc -O1 -g -std=c11 -fPIC -shared -fopenmp -ffp-contract=off -mfma -fno-fast-math -fno-finite-math-only \
    -fsanitize=address,undefined,float-cast-overflow -fno-sanitize-recover=all -fno-omit-frame-pointer \
    "$here/gs_oracle.c" -o "$out/libgs_oracle_san.so" -lm
cd "$here/.."
GS_ORACLE_LIB="$out/libgs_oracle_san.so" \
LD_PRELOAD="$(gcc -print-file-name=libasan.so) $(gcc -print-file-name=libubsan.so)" \
ASAN_OPTIONS=detect_leaks=0:abort_on_error=1 \
UBSAN_OPTIONS=print_stacktrace=1:halt_on_error=1 \
python -m pytest tests/test_oracle_bound.py tests/test_oracle_coverage.py tests/test_oracle_pipeline.py \
    -q -m "not gpu" -p no:cacheprovider "$@"
