#!/bin/sh
# Sanitizer runs of the host expert tier (host code only): builds the tier and its driver host_tier_check.cpp with
# ThreadSanitizer and with AddressSanitizer + UBSan (make tsan asan) and runs each twice: the serving cases (24
# jobs beside a thread that sets the mode and limit and reads the statistics; oversize jobs; a job republished
# while it is copied; a late answer) and the exit case (the process exits with the worker inside a job, the
# mailbox freed by an earlier-registered exit handler). Needs an AVX-512 (VBMI2, VNNI) host and gcc's sanitizer
# runtimes. Exits non-zero on a reported race, an invalid access or a failed check.
set -e
cd "$(dirname "$0")"
make -s tsan asan
for b in tsan asan; do
    TSAN_OPTIONS="halt_on_error=1 second_deadlock_stack=1" ASAN_OPTIONS="halt_on_error=1 detect_leaks=0" \
        ./_san/host_tier_$b
    TSAN_OPTIONS="halt_on_error=1" ASAN_OPTIONS="halt_on_error=1 detect_leaks=0" ./_san/host_tier_$b exit
    echo "sanitize_check: $b clean"
done
