#!/bin/bash
# Builds the host half of the round protocol (ipc_queue.cpp, aggregator.cpp)
# with g++ -fsanitize=thread, links the harness protocol_tsan.cpp, and runs
# it.  Output directory: $1 (default: a fresh temporary directory).  The
# aggregator source is compiled from a copy whose queue mapping is bound to
# the worker-side mapping of the same process, so both roles touch the
# shared words at one address (ThreadSanitizer tracks virtual addresses).
set -euo pipefail
here=$(cd "$(dirname "$0")" && pwd)
repo=$(cd "$here/../.." && pwd)
out=${1:-$(mktemp -d)}
mkdir -p "$out"
src=$repo/swarmlora_amd/csrc
sed 's/^swl::QueueMap g_agg_q;\(.*\)$/swl::QueueMap\& g_agg_q = swl::g_queue;\1/' "$src/aggregator.cpp" > "$out/aggregator_tsan.cpp"
if [ "${SWL_TSAN_PLANT:-0}" = "1" ]; then
  # planted mistake for the harness's own check (with the one below): the
  # barrier reads the ready set without acquire ordering
  sed -i 's/const Mask missing = active \& ~c->ready.load();/const Mask missing = active \& ~c->ready.load(std::memory_order_relaxed);/' \
      "$out/aggregator_tsan.cpp"
  grep -q 'ready.load(std::memory_order_relaxed)' "$out/aggregator_tsan.cpp"
fi
n=$(grep -c '^swl::QueueMap& g_agg_q = swl::g_queue;' "$out/aggregator_tsan.cpp" || true)
if [ "$n" != "1" ]; then echo "run_tsan.sh: aggregator.cpp no longer declares g_agg_q as expected" >&2; exit 3; fi
flags="-std=c++17 -O1 -g -fno-omit-frame-pointer -D__HIP_PLATFORM_AMD__ -I/opt/rocm/include -I$repo/include -I$src"
g++ $flags -fsanitize=thread -c "$out/aggregator_tsan.cpp" -o "$out/aggregator.o"
if [ "${SWL_TSAN_PLANT:-0}" = "1" ]; then
  # ... and the ring entry's ready flag is published without release
  # ordering, so nothing orders the worker's writes of the entry before the
  # aggregator's reads of it
  sed 's/cmd.ready.store(1, std::memory_order_release);/cmd.ready.store(1, std::memory_order_relaxed);/' \
      "$src/ipc_queue.cpp" > "$out/ipc_queue_planted.cpp"
  grep -q 'cmd.ready.store(1, std::memory_order_relaxed);' "$out/ipc_queue_planted.cpp"
  g++ $flags -fsanitize=thread -c "$out/ipc_queue_planted.cpp" -o "$out/ipc_queue.o"
else
  g++ $flags -fsanitize=thread -c "$src/ipc_queue.cpp" -o "$out/ipc_queue.o"
fi
g++ $flags -fsanitize=thread -c "$here/stubs.cpp" -o "$out/stubs.o"
g++ $flags -fsanitize=thread -c "$here/protocol_tsan.cpp" -o "$out/protocol_tsan.o"
g++ -fsanitize=thread "$out"/protocol_tsan.o "$out"/aggregator.o "$out"/ipc_queue.o "$out"/stubs.o \
    -L/opt/rocm/lib -lamdhip64 -Wl,-rpath,/opt/rocm/lib -lpthread -o "$out/protocol_tsan"
TSAN_OPTIONS="halt_on_error=0 exitcode=66 ${TSAN_OPTIONS:-}" "$out/protocol_tsan"
