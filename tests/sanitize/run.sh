#!/bin/bash
# CPU sanitizer run (host code only, no GPU): the oracle's C restatement and
# the host GGUF reader built with AddressSanitizer + UndefinedBehaviorSanitizer
# (gcc / g++, not hipcc).  1. the oracle's CPU tests against the instrumented
# oracle library (libasan preloaded into python); 2. the GGUF reader driver
# over well-formed, truncated and byte-flipped files.  Exits non-zero on any
# test failure or sanitizer report.  Outputs go to tests/sanitize/_build.
set -euo pipefail
HERE="$(cd "$(dirname "$0")" && pwd)"
ROOT="$(cd "$HERE/../.." && pwd)"
OUT="$HERE/_build"
mkdir -p "$OUT"
SAN="-fsanitize=address,undefined -fno-sanitize-recover=undefined -fno-omit-frame-pointer -g -O1"

gcc -std=c11 -fPIC -fopenmp -ffp-contract=off -fno-fast-math -Wall -Wextra $SAN -shared \
    -o "$OUT/libfuel_oracle_asan.so" "$ROOT/oracle/fuel_oracle.c" -lm
g++ -std=c++17 -Wall $SAN -o "$OUT/gguf_check" "$HERE/gguf_check.cpp" "$ROOT/fuel_amd/csrc/gguf.cpp"

export ASAN_OPTIONS=detect_leaks=0:abort_on_error=1
export UBSAN_OPTIONS=print_stacktrace=1:halt_on_error=1
LIBASAN="$(gcc -print-file-name=libasan.so)"
LIBUBSAN="$(gcc -print-file-name=libubsan.so)"

echo "== oracle CPU tests on the instrumented oracle"
(cd "$ROOT" && FUEL_ORACLE_LIB="$OUT/libfuel_oracle_asan.so" LD_PRELOAD="$LIBASAN:$LIBUBSAN" \
    python -m pytest -q -x -m "not gpu" -p no:cacheprovider tests/test_oracle_*.py 2>&1 | tail -3)

echo "== GGUF reader over well-formed, truncated and corrupted files"
rm -rf "$OUT/gguf_cases"
python "$HERE/make_gguf_cases.py" "$OUT/gguf_cases"
find "$OUT/gguf_cases" -name '*.gguf' -print0 | xargs -0 -n 200 "$OUT/gguf_check" > "$OUT/gguf_check.log"
echo "$(grep -c ': v' "$OUT/gguf_check.log") parsed, $(grep -c ': error' "$OUT/gguf_check.log") rejected, no sanitizer report"
