"""Host-side tests of the command ring / slot barrier protocol (no GPU).

Covers the failure cases the reference's barrier handles
(src/cpp_extensions/ext_aggregator.cpp:879-987, :1129-1160 and
ext_ipc_queue.cpp:272-402): eviction of a slot that never signals ready,
a mid-op leave, a full ring, validation before a ring entry is reserved, the
quit flag during an epoch wait, and commands of inactive slots being drained
and dropped.  The aggregator side is driven through the exported barrier
primitives, so every wait is bounded and no GPU work is involved.
"""

import ctypes
import multiprocessing as mp
import time

import pytest

from swarmlora_amd import _lib
from swarmlora_amd import ext_aggregator  # noqa: F401  (registers signatures)
from swarmlora_amd import ext_ipc_queue as extq

OP_QKV = 9


@pytest.fixture()
def queue():
    q = extq.create_queue(16, 16)
    extq.init_batch_control(8)
    L = _lib.load()
    _lib.check(L.swl_agg_attach_queue(q["shm_name"].encode(), 16))
    _lib.check(L.swl_agg_set_barrier_timeouts(60, 5))
    yield q
    extq.set_quit(0)
    _lib.check(L.swl_agg_set_barrier_timeouts(500, 10))
    extq.close_queue()


def _mask(slots):
    lo = hi = 0
    for s in slots:
        if s < 64:
            lo |= 1 << s
        else:
            hi |= 1 << (s - 64)
    return lo, hi


def _wait(slots):
    lo, hi = _mask(slots)
    clo, chi, cnt = ctypes.c_uint64(lo), ctypes.c_uint64(hi), ctypes.c_int(0)
    _lib.check(_lib.load().swl_agg_wait_for_slots(ctypes.byref(clo), ctypes.byref(chi), ctypes.byref(cnt)))
    return cnt.value, [s for s in range(128) if ((clo.value if s < 64 else chi.value) >> (s % 64)) & 1]


def _drain(slots, want):
    lo, hi = _mask(slots)
    arr = lambda t: (t * 128)()  # noqa: E731
    sids, wids, ops, lay = arr(ctypes.c_int32), arr(ctypes.c_int32), arr(ctypes.c_int32), arr(ctypes.c_int32)
    toks, keys, got = arr(ctypes.c_int64), arr(ctypes.c_uint64), ctypes.c_int(0)
    _lib.check(_lib.load().swl_agg_drain_commands(lo, hi, want, sids, wids, ops, lay, toks, keys, ctypes.byref(got)))
    return [(sids[i], wids[i], ops[i], lay[i], toks[i], keys[i]) for i in range(got.value)]


def _publish_active(slots):
    """What the main loop does at a token boundary: joins become active."""
    for s in slots:
        extq.slot_signal_join(s)


def test_layout_sizes():
    L = _lib.load()
    assert L.swl_q_command_bytes() == 128
    assert L.swl_q_control_bytes() % 64 == 0


def test_submit_validates_before_reserving(queue):
    for bad in [dict(slot_id=-1), dict(slot_id=128), dict(worker_id=-3), dict(worker_id=100001), dict(bx=0),
                dict(tx=70000)]:
        args = dict(op_type=OP_QKV, layer_idx=0, slot_id=1, worker_id=5, bx=1, tx=1, dx=4096, x_key=0, y0_key=0,
                    y1_key=0, y2_key=0, ticket_id=0)
        args.update(bad)
        with pytest.raises(RuntimeError):
            extq.submit_slot_command(**args)
    extq.submit_slot_command(OP_QKV, 3, 1, 5, 1, 2, 4096, 7, 0, 0, 0, 0)
    got = _drain([1], 1)
    assert got == [(1, 5, OP_QKV, 3, 2, 7)]  # the first entry is the valid one: nothing was reserved before


def test_ring_full(queue):
    for i in range(15):  # capacity 16 keeps one entry free
        extq.submit_slot_command(OP_QKV, 0, i % 8, 1, 1, 1, 4096, 0, 0, 0, 0, 0)
    with pytest.raises(RuntimeError, match="command ring buffer FULL"):
        extq.submit_slot_command(OP_QKV, 0, 0, 1, 1, 1, 4096, 0, 0, 0, 0, 0)
    assert len(_drain(list(range(8)), 15)) == 15
    extq.submit_slot_command(OP_QKV, 0, 0, 1, 1, 1, 4096, 0, 0, 0, 0, 0)  # space again


def test_wait_for_epoch_raises_on_quit(queue):
    extq.set_quit(1)
    with pytest.raises(RuntimeError, match="quit flag set"):
        extq.wait_for_epoch(extq.get_barrier_done_epoch())


def test_signal_done_advances_epoch_and_clears_ready(queue):
    ctrl_slots = [0, 1]
    cnt, active = _wait([])  # nothing active: returns immediately
    assert cnt == 0
    e0 = extq.get_barrier_done_epoch()
    extq.slot_signal_ready(0)
    extq.slot_signal_ready(1)
    cnt, active = _wait(ctrl_slots)
    assert cnt == 2 and active == [0, 1]
    _lib.check(_lib.load().swl_agg_signal_done())
    assert extq.get_barrier_done_epoch() == e0 + 1
    assert extq.wait_for_epoch(e0) == e0 + 1


def test_barrier_evicts_a_silent_slot(queue):
    extq.slot_signal_ready(0)
    extq.slot_signal_ready(2)
    t0 = time.time()
    cnt, active = _wait([0, 1, 2])  # slot 1 never signals
    assert time.time() - t0 < 5
    assert cnt == 2 and active == [0, 2]
    assert extq.is_slot_evicted(1) and not extq.is_slot_evicted(0)
    extq.clear_evicted_slot(1)
    assert not extq.is_slot_evicted(1)


def test_barrier_mid_op_leave(queue):
    extq.slot_signal_ready(0)
    extq.slot_signal_ready(1)
    extq.slot_signal_leave(2)
    cnt, active = _wait([0, 1, 2])
    assert cnt == 2 and active == [0, 1]
    assert not extq.is_slot_evicted(2)


def test_all_slots_leave(queue):
    extq.slot_signal_leave(4)
    cnt, active = _wait([4])
    assert cnt == 0 and active == []


def test_quit_ends_barrier_wait(queue):
    extq.set_quit(1)
    cnt, _ = _wait([3])
    assert cnt == -1


def test_drain_drops_commands_of_inactive_slots(queue):
    extq.submit_slot_command(OP_QKV, 0, 5, 9, 1, 1, 4096, 0, 0, 0, 0, 0)  # evicted slot's dangling command
    extq.submit_slot_command(OP_QKV, 0, 1, 2, 1, 1, 4096, 0, 0, 0, 0, 0)
    extq.submit_slot_command(OP_QKV, 0, 3, 4, 1, 1, 4096, 0, 0, 0, 0, 0)
    got = _drain([1, 3], 2)
    assert [g[0] for g in got] == [1, 3]


def _worker(shm_name, slot, worker_id, n_ops, out):
    from swarmlora_amd import ext_ipc_queue as q
    q.open_queue(shm_name, 16, 16)
    for op in range(n_ops):
        epoch = q.get_barrier_done_epoch()
        q.submit_slot_command(OP_QKV, op, slot, worker_id, 1, 1, 4096, 0, 0, 0, 0, 0)
        q.slot_signal_ready(slot)
        q.wait_for_epoch(epoch)
    out.put((worker_id, q.get_barrier_done_epoch()))


def test_multiprocess_lockstep_rounds(queue):
    """Three worker processes run 20 lock-step ops against this process's
    barrier: every op drains exactly one command per worker, in any order."""
    ctx = mp.get_context("spawn")
    out = ctx.Queue()
    n_ops = 20
    slots = [0, 3, 5]
    procs = [ctx.Process(target=_worker, args=(queue["shm_name"], s, 10 + s, n_ops, out)) for s in slots]
    for p in procs:
        p.start()
    try:
        for op in range(n_ops):
            deadline = time.time() + 60
            while True:
                cnt, active = _wait(slots)
                if cnt == 3:
                    break
                assert time.time() < deadline, "workers did not reach the barrier"
            cmds = _drain(slots, 3)
            assert sorted(c[0] for c in cmds) == slots
            assert all(c[3] == op for c in cmds)  # layer field carries the op index
            _lib.check(_lib.load().swl_agg_signal_done())
        res = [out.get(timeout=60) for _ in procs]
        assert sorted(r[0] for r in res) == [10, 13, 15]
        assert all(r[1] >= n_ops for r in res)
    finally:
        for p in procs:
            p.join(timeout=30)
            if p.is_alive():
                p.kill()


def _boundary(lo=0, hi=0):
    """The main loop's token boundary over the active set (lo, hi): leaves
    out, joins in, the result published; returns the active slots."""
    clo, chi, n = ctypes.c_uint64(lo), ctypes.c_uint64(hi), ctypes.c_int(0)
    _lib.check(_lib.load().swl_agg_token_boundary(ctypes.byref(clo), ctypes.byref(chi), ctypes.byref(n)))
    return [s for s in range(128) if ((clo.value if s < 64 else chi.value) >> (s % 64)) & 1]


def _tenant_killed_later(shm_name, slot, late_ready, out, cmd):
    """A worker that joins, runs op 0, goes silent for op 1 (the barrier
    evicts it), optionally signals ready late, and waits to be killed."""
    from swarmlora_amd import ext_ipc_queue as q
    q.open_queue(shm_name, 16, 16)
    q.slot_signal_join(slot)
    t0 = time.time()
    while not q.slot_is_active(slot):
        if time.time() - t0 > 60:
            out.put("never active")
            return
        time.sleep(0.001)
    epoch = q.get_barrier_done_epoch()
    q.submit_slot_command(OP_QKV, 0, slot, 77, 1, 1, 4096, 0, 0, 0, 0, 0)
    q.slot_signal_ready(slot)
    q.wait_for_epoch(epoch)
    out.put("op0")
    cmd.get(timeout=60)  # op 1 ran without it: evicted
    if late_ready:
        q.slot_signal_ready(slot)
    out.put("parked")
    time.sleep(600)


@pytest.mark.parametrize("late_ready", [False, True])
def test_worker_killed_with_its_slot_open(queue, late_ready):
    """Failure case of a worker SIGKILLed while its slot is open
    (ext_aggregator.cpp:215-227, aggregator.py:484-528): the silent slot is
    evicted by the barrier, the controller signals its leave and releases it
    at a token boundary, and the next tenant of the slot starts with clean
    barrier bits.  The dead tenant leaves an evicted bit (which would make
    the new tenant abort its request) and, if it signalled ready after the
    eviction, a ready bit that no signal_done clears any more (the slot is no
    longer active) and that would let the new tenant's first op run without
    its input.  The claim's scrub (swl_agg_scrub_slot, what claim_slot runs
    after winning the slot; the pool itself needs the GPU) clears both: the
    barrier then waits for the new tenant's own ready."""
    import os
    import signal
    from swarmlora_amd import ext_aggregator as agg
    ctx = mp.get_context("spawn")
    out, cmd = ctx.Queue(), ctx.Queue()
    slot = 3
    p = ctx.Process(target=_tenant_killed_later, args=(queue["shm_name"], slot, late_ready, out, cmd))
    p.start()
    try:
        active = []
        t0 = time.time()
        while slot not in active:
            assert time.time() - t0 < 120, "the worker never joined"
            active = _boundary()
            time.sleep(0.001)
        cnt, active = _wait([slot])  # op 0
        assert cnt == 1 and [c[0] for c in _drain([slot], 1)] == [slot]
        _lib.check(_lib.load().swl_agg_signal_done())
        assert out.get(timeout=60) == "op0"
        cnt, active = _wait([slot])  # op 1: the worker stays silent and is evicted
        assert cnt == 0 and active == [] and extq.is_slot_evicted(slot)
        _lib.check(_lib.load().swl_agg_signal_done())
        cmd.put("go")
        assert out.get(timeout=60) == "parked"
        os.kill(p.pid, signal.SIGKILL)
        p.join(timeout=30)
        assert p.exitcode == -signal.SIGKILL
        # the controller sees the dead worker: leave, then release at a token boundary
        extq.slot_signal_leave(slot)
        assert _boundary(1 << slot) == []
        if late_ready:
            # the late ready bit survived: a barrier over the slot would pass at once
            cnt, active = _wait([slot])
            assert cnt == 1 and active == [slot]
        # the next claim of the slot scrubs its bits; the new tenant joins
        agg.scrub_slot(slot)
        assert not extq.is_slot_evicted(slot)
        extq.slot_signal_join(slot)
        assert _boundary() == [slot]
        t0 = time.time()
        cnt, active = _wait([slot])  # no stale ready: the barrier waits for the new tenant (and evicts it here)
        assert cnt == 0 and time.time() - t0 >= 0.05
        agg.scrub_slot(slot)
        extq.slot_signal_ready(slot)  # the new tenant's own ready
        cnt, active = _wait([slot])
        assert cnt == 1 and active == [slot] and not extq.is_slot_evicted(slot)
        _lib.check(_lib.load().swl_agg_signal_done())
    finally:
        if p.is_alive():
            p.kill()
            p.join(timeout=30)
        _boundary()  # drop what the test left in the join / leave sets
