"""ThreadSanitizer run of the shared-memory round protocol (CPU only).

tests/tsan/run_tsan.sh builds the host half of the protocol
(csrc/ipc_queue.cpp, csrc/aggregator.cpp) with g++ -fsanitize=thread and runs
tests/tsan/protocol_tsan.cpp: worker threads and an aggregator thread go
through lock-step ops with a late join, leaves at a token boundary and in
the middle of an op, an evicted slot and ring wrap-around, over one mapping
of the segment.  The reference's layout and waits are ipc_types.h:105-146
and ext_ipc_queue.cpp:272-402.

The second test plants a real ordering mistake in copies of the sources (the
ready set read without acquire and the ring entry published without
release) and checks that the same harness reports data races, so a clean
run means the accesses were seen.
"""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SCRIPT = os.path.join(HERE, "tsan", "run_tsan.sh")

pytestmark = [
    pytest.mark.skipif(not os.path.exists(SCRIPT), reason="ThreadSanitizer harness not present"),
    pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available"),
    pytest.mark.skipif(not os.path.exists("/opt/rocm/lib/libamdhip64.so"), reason="HIP runtime library absent"),
]


def _run(tmp_path, plant):
    env = dict(os.environ, SWL_TSAN_PLANT="1" if plant else "0")
    p = subprocess.run(["bash", SCRIPT, str(tmp_path)], env=env, capture_output=True, text=True, timeout=600)
    return p.returncode, p.stdout + p.stderr


def test_protocol_is_race_free_under_tsan(tmp_path):
    rc, out = _run(tmp_path, plant=False)
    assert "WARNING: ThreadSanitizer" not in out, out[-4000:]
    assert rc == 0, out[-4000:]
    assert "all invariants held" in out
    assert "EVICTING stuck slot" in out and "Mid-op slot leave" in out


def test_tsan_harness_reports_a_planted_race(tmp_path):
    rc, out = _run(tmp_path, plant=True)
    assert "WARNING: ThreadSanitizer: data race" in out, out[-4000:]
    assert rc != 0
