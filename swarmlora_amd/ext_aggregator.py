"""Aggregator: slot pool, fused weights, batched rounds and the main loop.

Drop-in for the reference's ``ext_aggregator`` pybind module
(src/cpp_extensions/ext_aggregator.cpp:1436-1517): same function names,
argument names, return dictionaries and error texts; errors raise
RuntimeError.  Everything runs in libswl.so (swarmlora_amd/csrc/
aggregator.cpp) on its own HIP kernels; ``aggregator_main_loop_slots``
releases the GIL for its whole duration (ctypes drops it around the call).

Additions beyond the reference's API (its workers compute their own LoRA
delta): ``register_adapter`` / ``clear_adapters`` fill an adapter pool whose
deltas the rounds add during the scatter (a command selects pool adapter
``a`` with ``x_key = a + 1``), and ``execute_round`` / ``slot_tensors`` run a
round and expose slot buffers to in-process callers.
"""

import ctypes
from typing import Optional, Sequence

import torch

from . import _lib
from ._lib import P_i32, P_i64, PoolStatus, c_f32, c_i64, c_int, c_u64, c_vp

OP_O_PROJ = 3
OP_DOWN_PROJ = 6
OP_QKV_FUSED = 9
OP_GATE_UP_FUSED = 10
OP_EMBED = 11
OP_LM_HEAD = 12
OP_SET_SAMPLING = 13
MAX_SLOTS = 128

_P_size = ctypes.POINTER(ctypes.c_size_t)
_P_u64 = ctypes.POINTER(c_u64)

_lib.register_signatures({
    "swl_agg_init_slot_pool": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, _P_size, _P_size]),
    "swl_agg_claim_slot": (c_int, [c_int, ctypes.POINTER(c_int), ctypes.c_char_p, ctypes.c_char_p, _P_size,
                                   _P_size]),
    "swl_agg_release_slot": (c_int, [c_int, c_int]),
    "swl_agg_get_slot_owner": (c_int, [c_int]),
    "swl_agg_pool_status": (c_int, [ctypes.POINTER(PoolStatus)]),
    "swl_agg_cleanup_slot_pool": (c_int, []),
    "swl_agg_slot_buffers": (c_int, [c_int, ctypes.POINTER(c_vp), ctypes.POINTER(c_vp)]),
    "swl_agg_begin": (c_int, [c_int, c_int]),
    "swl_agg_set_layer": (c_int, [c_int, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_vp, c_i64,
                                  c_vp, c_vp, c_i64, c_i64]),
    "swl_agg_finalize": (c_int, []),
    "swl_agg_set_embed_lm_head": (c_int, [c_vp, c_vp, c_i64, c_i64]),
    "swl_agg_attach_queue": (c_int, [ctypes.c_char_p, c_int]),
    "swl_agg_scrub_slot": (c_int, [c_int]),
    "swl_agg_token_boundary": (c_int, [ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64),
                                       ctypes.POINTER(c_int)]),
    "swl_agg_register_adapter": (c_int, [c_int, c_int, c_int, c_vp, ctypes.POINTER(c_vp), c_int, c_int, c_f32]),
    "swl_agg_clear_adapters": (c_int, []),
    "swl_agg_execute_round": (c_int, [c_int, c_int, c_int, P_i32, P_i32, P_i64, P_i32, c_vp]),
    "swl_agg_wait_for_slots": (c_int, [_P_u64, _P_u64, ctypes.POINTER(c_int)]),
    "swl_agg_signal_done": (c_int, []),
    "swl_agg_drain_commands": (c_int, [c_u64, c_u64, c_int, P_i32, P_i32, P_i32, P_i32, P_i64, _P_u64,
                                       ctypes.POINTER(c_int)]),
    "swl_agg_set_barrier_timeouts": (c_int, [c_int, c_int]),
    "swl_agg_main_loop": (c_int, [c_int, c_int]),
    "swl_agg_take_seq_timeouts": (c_int, [ctypes.POINTER(ctypes.c_int32), c_int]),
})

# Tensors whose memory the library points at (o/down weights, biases, embed
# and LM-head tables): kept alive for the process lifetime, as the reference
# keeps its detach()-shared tensors.  Pooled adapters are kept per pool entry
# and released when the entry is replaced or the pool cleared.
_keep = []
_adapter_keep = {}
_pool_info = {}


def _L():
    return _lib.load()


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _weight(t, name):
    if not isinstance(t, torch.Tensor) or not t.is_cuda or t.dtype != torch.bfloat16:
        raise RuntimeError(f"{name} must be a bfloat16 GPU tensor")
    return t.contiguous()


def _opt_bias(t, name):
    if t is None or t.numel() == 0:
        return None
    return _weight(t, name)


# ------------------------------------------------------------------ weights
def init_aggregator_begin(num_layers, device_index):
    _lib.check(_L().swl_agg_begin(int(num_layers), int(device_index)))


def init_aggregator_layer(layer_idx, q_weight, k_weight, v_weight, o_weight, o_bias, gate_weight, up_weight,
                          down_weight, down_bias):
    q, k, v = (_weight(t, n) for t, n in ((q_weight, "q_weight"), (k_weight, "k_weight"), (v_weight, "v_weight")))
    o = _weight(o_weight, "o_weight")
    g, u = _weight(gate_weight, "gate_weight"), _weight(up_weight, "up_weight")
    d = _weight(down_weight, "down_weight")
    ob, db = _opt_bias(o_bias, "o_bias"), _opt_bias(down_bias, "down_bias")
    hidden = q.shape[1]
    inter = g.shape[0]
    for t, nm in ((k, "k_weight"), (v, "v_weight"), (o, "o_weight"), (g, "gate_weight"), (u, "up_weight")):
        if t.shape[1] != hidden:
            raise RuntimeError(f"init_aggregator_layer: {nm} input dim {t.shape[1]} != hidden {hidden}")
    if d.shape != (hidden, inter) or u.shape[0] != inter or o.shape[0] != hidden:
        raise RuntimeError("init_aggregator_layer: o/down/up shapes do not match hidden/intermediate sizes")
    _lib.check(_L().swl_agg_set_layer(int(layer_idx), _ptr(q), q.shape[0], _ptr(k), k.shape[0], _ptr(v), v.shape[0],
                                      _ptr(o), _ptr(ob), _ptr(g), g.shape[0], _ptr(u), u.shape[0], _ptr(d), _ptr(db),
                                      hidden, inter))
    _keep.extend(t for t in (o, ob, d, db) if t is not None)


def init_aggregator_finalize():
    _lib.check(_L().swl_agg_finalize())


def init_aggregator_queue(shm_name, capacity):
    _lib.check(_L().swl_agg_attach_queue(str(shm_name).encode(), int(capacity)))


def init_embed_lm_head_weights(embed_weight, lm_head_weight):
    e = _weight(embed_weight, "embed_weight")
    h = _weight(lm_head_weight, "lm_head_weight")
    if e.shape != h.shape:
        raise RuntimeError("init_embed_lm_head_weights: embed and lm_head must both be [vocab, hidden]")
    _lib.check(_L().swl_agg_set_embed_lm_head(_ptr(e), _ptr(h), e.shape[0], e.shape[1]))
    _keep.extend([e, h])


# ---------------------------------------------------------------- slot pool
def init_slot_pool(num_slots, device_index, hidden_dim, intermediate_dim, num_kv_heads, head_dim, max_seq_per_step,
                   dtype_size):
    ins, outs = ctypes.c_size_t(0), ctypes.c_size_t(0)
    _lib.check(_L().swl_agg_init_slot_pool(int(num_slots), int(device_index), int(hidden_dim), int(intermediate_dim),
                                           int(num_kv_heads), int(head_dim), int(max_seq_per_step), int(dtype_size),
                                           ctypes.byref(ins), ctypes.byref(outs)))
    _pool_info.update(device=int(device_index), input_buffer_size=ins.value, output_buffer_size=outs.value)
    return {"num_slots": int(num_slots), "input_buffer_size": ins.value, "output_buffer_size": outs.value}


def claim_slot(worker_id):
    sid = c_int(-1)
    hin = ctypes.create_string_buffer(64)
    hout = ctypes.create_string_buffer(64)
    ins, outs = ctypes.c_size_t(0), ctypes.c_size_t(0)
    _lib.check(_L().swl_agg_claim_slot(int(worker_id), ctypes.byref(sid), hin, hout, ctypes.byref(ins),
                                       ctypes.byref(outs)))
    return {"slot_id": sid.value, "worker_id": int(worker_id), "input_handle": hin.raw, "output_handle": hout.raw,
            "input_buffer_size": ins.value, "output_buffer_size": outs.value}


def scrub_slot(slot_id):
    """claim_slot's reset of a slot's ready / evicted bits for its next owner
    (ext_aggregator.cpp:223-227); claim_slot runs it itself."""
    _lib.check(_L().swl_agg_scrub_slot(int(slot_id)))


def release_slot(slot_id, worker_id):
    _lib.check(_L().swl_agg_release_slot(int(slot_id), int(worker_id)))


def get_slot_owner(slot_id):
    return int(_L().swl_agg_get_slot_owner(int(slot_id)))


def get_slot_pool_status():
    st = PoolStatus()
    _lib.check(_L().swl_agg_pool_status(ctypes.byref(st)))
    free_count = bin(st.free_lo).count("1") + bin(st.free_hi).count("1")
    active_count = bin(st.active_lo).count("1") + bin(st.active_hi).count("1")
    return {"initialized": bool(st.initialized), "num_slots": st.num_slots, "free_mask_lo": st.free_lo,
            "free_mask_hi": st.free_hi, "active_mask_lo": st.active_lo, "active_mask_hi": st.active_hi,
            "free_count": free_count, "active_count": active_count, "active_slot_count": st.active_slot_count,
            "slot_owners": [st.owners[i] for i in range(st.num_slots)]}


def cleanup_slot_pool():
    _lib.check(_L().swl_agg_cleanup_slot_pool())


# ---------------------------------------------------------------- main loop
def aggregator_main_loop_slots(num_slots, dtype_code):
    """Blocks until the queue's quit flag is set (GIL released)."""
    _lib.check(_L().swl_agg_main_loop(int(num_slots), int(dtype_code)))


def export_weight_ipc_handles():
    raise RuntimeError("export_weight_ipc_handles: donor weight transfer between aggregators is a multi-GPU "
                       "feature and is not part of this single-GPU build")


def import_weights_from_ipc(handles_dict, target_device_index):
    raise RuntimeError("import_weights_from_ipc: donor weight transfer between aggregators is a multi-GPU "
                       "feature and is not part of this single-GPU build")


# ------------------------------------------------------ additions (pool/run)
class _DeviceArray:
    """__cuda_array_interface__ view of library-owned device memory."""

    def __init__(self, ptr, shape, typestr):
        self.__cuda_array_interface__ = {"data": (ptr, False), "shape": tuple(shape), "typestr": typestr,
                                         "version": 3, "strides": None}


def slot_tensors(slot_id, dtype=torch.bfloat16):
    """(input, output) torch views of slot `slot_id`'s buffers (flat, `dtype`)."""
    pin, pout = c_vp(), c_vp()
    _lib.check(_L().swl_agg_slot_buffers(int(slot_id), ctypes.byref(pin), ctypes.byref(pout)))
    esz = torch.empty(0, dtype=dtype).element_size()
    typestr = {torch.bfloat16: "<V2", torch.int64: "<i8", torch.float32: "<f4"}[dtype]
    dev = torch.device("cuda", _pool_info.get("device", 0))
    views = []
    for p, nbytes in ((pin.value, _pool_info["input_buffer_size"]), (pout.value, _pool_info["output_buffer_size"])):
        if dtype == torch.bfloat16:
            raw = torch.as_tensor(_DeviceArray(p, (nbytes // 2,), "<i2"), device=dev)
            views.append(raw.view(torch.bfloat16))
        else:
            views.append(torch.as_tensor(_DeviceArray(p, (nbytes // esz,), typestr), device=dev))
    return views[0], views[1]


def register_adapter(adapter_id, layer_idx, op_type, lora_a, lora_b: Sequence[torch.Tensor], scale):
    """Pool adapter `adapter_id` for (layer_idx, op_type).  lora_a: bf16
    [nblk*rank, in] (the blocks' lora_A stacked); lora_b[j]: bf16 [cols_j, rank]."""
    a = _weight(lora_a, "lora_a")
    bs = [_weight(b, f"lora_b[{j}]") for j, b in enumerate(lora_b)]
    rank = bs[0].shape[1]
    if a.shape[0] != rank * len(bs) or any(b.shape[1] != rank for b in bs):
        raise RuntimeError("register_adapter: lora_a must be [nblk*rank, in] and every lora_b [cols, rank]")
    arr = (c_vp * len(bs))(*[b.data_ptr() for b in bs])
    key = (int(adapter_id), int(layer_idx), int(op_type))
    old = _adapter_keep.get(key)
    if old is not None and any(t.data_ptr() != n.data_ptr() for t, n in zip(old, [a, *bs])):
        torch.cuda.synchronize()  # rounds already queued may still read the tensors being replaced
    _lib.check(_L().swl_agg_register_adapter(int(adapter_id), int(layer_idx), int(op_type), a.data_ptr(), arr,
                                             len(bs), int(rank), float(scale)))
    _adapter_keep[key] = [a, *bs]


def take_seq_timeouts():
    """Slots whose GPU-ordered input did not arrive within the aggregator
    stream's wait limit since the last call (the main loop evicts them)."""
    arr = (ctypes.c_int32 * 128)()
    n = _L().swl_agg_take_seq_timeouts(arr, 128)
    return list(arr[:min(n, 128)])


def clear_adapters():
    _lib.check(_L().swl_agg_clear_adapters())
    if _adapter_keep:
        if torch.cuda.is_available():
            torch.cuda.synchronize()
        _adapter_keep.clear()


def execute_round(op_type, layer_idx, slot_ids, worker_ids, tokens, adapter_ids: Optional[Sequence[int]] = None,
                  stream: Optional[torch.cuda.Stream] = None):
    """One batched round over the slot pool on `stream` (default: torch's
    current stream): execute_batched_gemm_slots plus pooled LoRA deltas."""
    n = len(slot_ids)
    s_arr = (ctypes.c_int32 * n)(*slot_ids)
    w_arr = (ctypes.c_int32 * n)(*worker_ids) if worker_ids is not None else None
    t_arr = (ctypes.c_int64 * n)(*tokens)
    a_arr = (ctypes.c_int32 * n)(*adapter_ids) if adapter_ids is not None else None
    st = stream if stream is not None else torch.cuda.current_stream()
    _lib.check(_L().swl_agg_execute_round(int(op_type), int(layer_idx), n, s_arr, w_arr, t_arr, a_arr,
                                          c_vp(st.cuda_stream)))
