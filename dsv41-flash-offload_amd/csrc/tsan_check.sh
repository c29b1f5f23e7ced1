#!/bin/sh
# ThreadSanitizer run of the host expert tier (host code only): builds the tier and its driver with
# -fsanitize=thread (make tsan) and runs it: the mailbox worker serving jobs while another thread sets the mode and
# the limit and reads the statistics, then the synchronous forward on the pool. Needs an AVX-512 (VBMI2, VNNI) host
# and gcc's TSan runtime. Exits non-zero on a reported race or a failed check.
set -e
cd "$(dirname "$0")"
make -s tsan
TSAN_OPTIONS="halt_on_error=1 second_deadlock_stack=1" ./_tsan/host_tier_tsan
echo "tsan_check: clean"
