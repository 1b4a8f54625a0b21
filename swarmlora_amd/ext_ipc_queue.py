"""Shared-memory command queue and slot barrier.

Drop-in for the reference's ``ext_ipc_queue`` pybind module
(src/cpp_extensions/ext_ipc_queue.cpp:413-483): same function names, argument
names, return values and error texts; errors raise RuntimeError.  The
protocol runs in libswl.so (swarmlora_amd/csrc/ipc_queue.cpp).
"""

import ctypes

from . import _lib
from ._lib import c_f32, c_i64, c_int, c_u64

_lib.register_signatures({
    "swl_q_create": (c_int, [c_int, c_int, ctypes.c_char_p, c_int]),
    "swl_q_open": (c_int, [ctypes.c_char_p, c_int, c_int]),
    "swl_q_close": (c_int, []),
    "swl_q_init_batch_control": (c_int, [c_int]),
    "swl_q_set_quit": (c_int, [c_int]),
    "swl_q_set_pending_sampling": (c_int, [c_int, c_int, c_f32, c_int, c_f32]),
    "swl_q_signal_join": (c_int, [c_int]),
    "swl_q_signal_leave": (c_int, [c_int]),
    "swl_q_signal_ready": (c_int, [c_int]),
    "swl_q_wait_for_epoch": (c_int, [c_i64, ctypes.POINTER(c_i64)]),
    "swl_q_slot_is_active": (c_int, [c_int]),
    "swl_q_is_slot_evicted": (c_int, [c_int]),
    "swl_q_clear_evicted_slot": (c_int, [c_int]),
    "swl_q_get_epoch": (c_i64, []),
    "swl_q_submit": (c_int, [c_int, c_int, c_int, c_int, c_i64, c_i64, c_i64, c_u64, c_u64, c_u64, c_u64, c_int]),
    "swl_q_submit_seq": (c_int, [c_int, c_int, c_int, c_int, c_i64, c_i64, c_i64, c_u64, c_u64, c_u64, c_u64, c_int,
                                 c_u64]),
    "swl_q_submit_seq_ex": (c_int, [c_int, c_int, c_int, c_int, c_i64, c_i64, c_i64, c_u64, c_u64, c_u64, c_u64,
                                    c_int, c_u64, c_int]),
    "swl_q_control_bytes": (ctypes.c_size_t, []),
    "swl_q_command_bytes": (ctypes.c_size_t, []),
})


def _L():
    return _lib.load()


def create_queue(capacity, max_tickets):
    buf = ctypes.create_string_buffer(256)
    _lib.check(_L().swl_q_create(int(capacity), int(max_tickets), buf, len(buf)))
    return {"shm_name": buf.value.decode(), "capacity": int(capacity), "max_tickets": int(max_tickets)}


def open_queue(shm_name, capacity, max_tickets):
    _lib.check(_L().swl_q_open(str(shm_name).encode(), int(capacity), int(max_tickets)))
    return {"capacity": int(capacity), "max_tickets": int(max_tickets)}


def close_queue():
    """Unmap this process's queue (unlinking it if this process created it)."""
    _lib.check(_L().swl_q_close())


def init_batch_control(num_slots):
    _lib.check(_L().swl_q_init_batch_control(int(num_slots)))


def set_quit(value):
    _lib.check(_L().swl_q_set_quit(int(value)))


def slot_set_pending_sampling(slot_id, do_sample, temperature, top_k, top_p):
    _lib.check(_L().swl_q_set_pending_sampling(int(slot_id), 1 if do_sample else 0, float(temperature),
                                               int(top_k), float(top_p)))


def slot_signal_join(slot_id):
    _lib.check(_L().swl_q_signal_join(int(slot_id)))


def slot_signal_leave(slot_id):
    _lib.check(_L().swl_q_signal_leave(int(slot_id)))


def slot_signal_ready(slot_id):
    _lib.check(_L().swl_q_signal_ready(int(slot_id)))


def wait_for_epoch(expected_epoch):
    out = c_i64(0)
    _lib.check(_L().swl_q_wait_for_epoch(int(expected_epoch), ctypes.byref(out)))
    return out.value


def slot_is_active(slot_id):
    return bool(_L().swl_q_slot_is_active(int(slot_id)))


def get_barrier_done_epoch():
    return int(_L().swl_q_get_epoch())


def is_slot_evicted(slot_id):
    return bool(_L().swl_q_is_slot_evicted(int(slot_id)))


def clear_evicted_slot(slot_id):
    _lib.check(_L().swl_q_clear_evicted_slot(int(slot_id)))


def submit_slot_command(op_type, layer_idx, slot_id, worker_id, bx, tx, dx, x_key, y0_key, y1_key, y2_key,
                        ticket_id, in_seq=0, out_host=False):
    """in_seq > 0 (an addition): the command is GPU-ordered -- the
    aggregator's stream waits for the slot's input sequence word to reach
    in_seq (ext_unified_barrier.input_seq after a GPU-ordered prepare).
    out_host (with in_seq): the worker reads the outputs once done is
    signalled, without a wait on its stream, so the aggregator finishes the
    round on its stream before signalling."""
    if in_seq:
        _lib.check(_L().swl_q_submit_seq_ex(int(op_type), int(layer_idx), int(slot_id), int(worker_id), int(bx),
                                            int(tx), int(dx), int(x_key), int(y0_key), int(y1_key), int(y2_key),
                                            int(ticket_id), int(in_seq), 1 if out_host else 0))
        return
    _lib.check(_L().swl_q_submit(int(op_type), int(layer_idx), int(slot_id), int(worker_id), int(bx), int(tx),
                                 int(dx), int(x_key), int(y0_key), int(y1_key), int(y2_key), int(ticket_id)))
