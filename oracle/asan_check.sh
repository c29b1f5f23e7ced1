#!/bin/sh
# Sanitizer run of the CPU oracle and of the reference kernel the golden writer calls (host code only):
# builds both with AddressSanitizer + UndefinedBehaviorSanitizer (make asan), then runs the oracle's tests and the
# golden writer in check mode (every fixture recomputed and compared bit for bit, nothing written) against them.
# Run from anywhere; needs gcc's sanitizer runtimes.
set -e
cd "$(dirname "$0")/.."
make -s -C oracle asan
RT="$(gcc -print-file-name=libasan.so) $(gcc -print-file-name=libubsan.so)"
export ASAN_OPTIONS=detect_leaks=0:abort_on_error=1
export UBSAN_OPTIONS=print_stacktrace=1:halt_on_error=1
LD_PRELOAD="$RT" MM_ORACLE_LIB="$PWD/oracle/_asan/libmmoracle.so" python -m pytest -q -x -p no:cacheprovider \
    tests/test_oracle.py tests/test_ec.py
if [ -f oracle/_asan/libftref.so ]; then
    LD_PRELOAD="$RT" MM_REF_LIB="$PWD/oracle/_asan/libftref.so" python tests/golden/make_golden.py --check
fi
echo "asan_check: clean"
