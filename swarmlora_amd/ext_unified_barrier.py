"""Worker-side slot manager: maps aggregator slot buffers via HIP IPC handles.

Drop-in for the reference's ``ext_unified_barrier`` pybind module
(src/cpp_extensions/ext_unified_barrier.cpp:562-630): same function names,
arguments, return values and error texts; errors raise RuntimeError.  Copies
run on torch's current stream of the worker device; ``get_outputs_slot`` and
``get_embeddings_slot`` return fresh worker-owned tensors (callers mutate
them in place), never views of the slot buffer.
"""

import ctypes
from typing import List, Sequence

import torch

from . import _lib
from ._lib import c_i64, c_int, c_vp

OP_O_PROJ = 3
OP_DOWN_PROJ = 6
OP_QKV_FUSED = 9
OP_GATE_UP_FUSED = 10
OP_EMBED = 11
OP_LM_HEAD = 12
OP_SET_SAMPLING = 13

_P_i64 = ctypes.POINTER(c_i64)
_P_size = ctypes.POINTER(ctypes.c_size_t)

_lib.register_signatures({
    "swl_w_init": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "swl_w_open_slot": (c_int, [c_int, ctypes.c_char_p, ctypes.c_size_t, ctypes.c_char_p, ctypes.c_size_t,
                                ctypes.c_size_t, ctypes.c_size_t]),
    "swl_w_close_slot": (c_int, [c_int]),
    "swl_w_prepare_input": (c_int, [c_int, c_vp, c_i64, c_i64, c_i64, ctypes.c_size_t, c_vp]),
    "swl_w_slot_shape": (c_int, [c_int, _P_i64, _P_i64, _P_i64]),
    "swl_w_slot_sizes": (c_int, [c_int, _P_size, _P_size]),
    "swl_w_copy_output": (c_int, [c_int, c_vp, ctypes.c_size_t, c_vp]),
    "swl_w_read_output": (c_int, [c_int, c_vp, c_i64, c_vp, c_vp, c_vp]),
    "swl_w_read_output_norm": (c_int, [c_int, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, ctypes.c_float,
                                       c_int, c_vp]),
    "swl_w_read_output_silu": (c_int, [c_int, c_vp, c_i64, c_i64, c_i64, c_vp, c_int, c_vp]),
    "swl_w_submit_staged_input": (c_int, [c_int, c_i64, c_i64, c_i64, c_vp]),
    "swl_w_stage_input": (c_int, [c_int, c_i64, c_i64, c_i64, ctypes.POINTER(c_vp)]),
    "swl_w_prepare_token_ids": (c_int, [c_int, c_vp, c_i64, c_i64, c_vp]),
    "swl_w_prepare_hidden_lm": (c_int, [c_int, c_vp, c_i64, c_i64, c_i64, ctypes.c_size_t, c_vp]),
    "swl_w_get_next_token": (c_int, [c_int, _P_i64, c_vp]),
    "swl_w_cleanup": (c_int, []),
    "swl_w_set_gpu_ordered": (c_int, [c_int]),
    "swl_w_input_seq": (c_int, [c_int, ctypes.POINTER(ctypes.c_uint64)]),
})

_state = {"device": 0, "hidden_dim": 0}


def _L():
    return _lib.load()


if hasattr(torch._C, "_cuda_getCurrentRawStream"):
    def _stream():  # the raw handle, without building a Stream object
        return c_vp(torch._C._cuda_getCurrentRawStream(_state["device"]))
else:
    def _stream():
        return c_vp(torch.cuda.current_stream(_state["device"]).cuda_stream)


def _shape(slot_id):
    bx, tx, dx = c_i64(0), c_i64(0), c_i64(0)
    _lib.check(_L().swl_w_slot_shape(int(slot_id), ctypes.byref(bx), ctypes.byref(tx), ctypes.byref(dx)))
    return bx.value, tx.value, dx.value


def init_worker_slot_manager(worker_id, worker_device, aggregator_device, hidden_dim, intermediate_dim, qkv_dim):
    _state.update(device=int(worker_device), hidden_dim=int(hidden_dim))
    _lib.check(_L().swl_w_init(int(worker_id), int(worker_device), int(aggregator_device), int(hidden_dim),
                               int(intermediate_dim), int(qkv_dim)))


def open_slot(slot_id, input_handle, output_handle, input_buffer_size, output_buffer_size):
    hin, hout = bytes(input_handle), bytes(output_handle)
    _lib.check(_L().swl_w_open_slot(int(slot_id), hin, len(hin), hout, len(hout), int(input_buffer_size),
                                    int(output_buffer_size)))


def close_slot(slot_id):
    _lib.check(_L().swl_w_close_slot(int(slot_id)))


def _device_tensor(t, name):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor")
    return t.contiguous()


def prepare_input_slot(slot_id, op_type, input):
    if not isinstance(input, torch.Tensor) or input.dim() != 3:
        raise RuntimeError("Input must be 3D [B, T, D]")
    x = _device_tensor(input, "input")
    b, t, d = x.shape
    _lib.check(_L().swl_w_prepare_input(int(slot_id), x.data_ptr(), b, t, d, x.element_size(), _stream()))


def get_outputs_slot(slot_id, out_dims: Sequence[int], input_template) -> List[torch.Tensor]:
    bx, tx, _ = _shape(slot_id)
    dims = [int(d) for d in out_dims]
    total = sum(dims)
    out = torch.empty(bx, tx, total, dtype=input_template.dtype, device=input_template.device)
    _lib.check(_L().swl_w_copy_output(int(slot_id), out.data_ptr(), out.numel() * out.element_size(), _stream()))
    if len(dims) > 1:
        return list(out.split(dims, dim=-1))
    return [out]


def read_outputs_slot(slot_id, out_dims: Sequence[int], input_template, delta=None, residual=None):
    """get_outputs_slot with the adds its caller makes next, in one launch:
    residual + (output + delta), bf16 roundings as torch's two adds; delta
    and residual are [B, T, sum(out_dims)] bf16 or None (an addition: the
    reference copies, then adds with torch).  Returns the same split views."""
    bx, tx, _ = _shape(slot_id)
    dims = [int(d) for d in out_dims]
    total = sum(dims)
    out = torch.empty(bx, tx, total, dtype=input_template.dtype, device=input_template.device)
    ptrs = []
    for name, t in (("delta", delta), ("residual", residual)):
        if t is None:
            ptrs.append(None)
            continue
        if (t.dtype != torch.bfloat16 or out.dtype != torch.bfloat16 or tuple(t.shape) != tuple(out.shape)
                or not t.is_contiguous()):
            raise RuntimeError(f"read_outputs_slot: {name} must be a contiguous bf16 [B, T, {total}] tensor")
        ptrs.append(t.data_ptr())
    _lib.check(_L().swl_w_read_output(int(slot_id), out.data_ptr(), out.numel(), ptrs[0], ptrs[1], _stream()))
    if len(dims) > 1:
        return list(out.split(dims, dim=-1))
    return [out]


def _bf16_operand(t, shape, name):
    if t is None:
        return None
    if t.dtype != torch.bfloat16 or tuple(t.shape) != tuple(shape) or not t.is_contiguous() or t.data_ptr() % 16:
        raise RuntimeError(f"read_outputs: {name} must be a contiguous, 16-byte aligned bf16 {list(shape)} tensor")
    return t.data_ptr()


def read_outputs_norm_slot(slot_id, out_dim, input_template, delta, residual, weight, eps, stage=False):
    """An O or Down round's output read with the worker's adds and the next
    LlamaRMSNorm in one launch (an addition): returns (h, norm(h) * weight),
    h = residual + (output + delta), [B, T, out_dim] each; out_dim a
    multiple of 8.  stage: norm(h) is also written into the slot's input
    buffer as the next round's input (submit_staged_input_slot)."""
    bx, tx, _ = _shape(slot_id)
    d = int(out_dim)
    shape = (bx, tx, d)
    h = torch.empty(shape, dtype=torch.bfloat16, device=input_template.device)
    n = torch.empty_like(h)
    if weight.dtype != torch.bfloat16 or weight.numel() != d or not weight.is_contiguous() or weight.data_ptr() % 16:
        raise RuntimeError("read_outputs_norm_slot: weight must be a contiguous, aligned bf16 [out_dim] tensor")
    _lib.check(_L().swl_w_read_output_norm(int(slot_id), h.data_ptr(), n.data_ptr(), bx, tx, d,
                                           _bf16_operand(delta, shape, "delta"),
                                           _bf16_operand(residual, shape, "residual"), weight.data_ptr(),
                                           float(eps), 1 if stage else 0, _stream()))
    return h, n


def read_outputs_silu_slot(slot_id, inter, input_template, delta=None, stage=False):
    """A Gate+Up round's output read (gate | up, plus the fused delta) and
    F.silu(gate) * up in one launch (an addition): [B, T, inter]; stage as
    read_outputs_norm_slot."""
    bx, tx, _ = _shape(slot_id)
    i = int(inter)
    act = torch.empty(bx, tx, i, dtype=torch.bfloat16, device=input_template.device)
    _lib.check(_L().swl_w_read_output_silu(int(slot_id), act.data_ptr(), bx, tx, i,
                                           _bf16_operand(delta, (bx, tx, 2 * i), "delta"), 1 if stage else 0,
                                           _stream()))
    return act


def submit_staged_input_slot(slot_id, input):
    """prepare_input_slot for an input a fused read already staged in the
    slot's input buffer (an addition): `input` is that read's result; its
    shape is checked against the staged rows, nothing is copied."""
    b, t, d = input.shape
    _lib.check(_L().swl_w_submit_staged_input(int(slot_id), b, t, d, _stream()))


class _DeviceArray:
    """__cuda_array_interface__ view of the slot's mapped input buffer."""

    def __init__(self, ptr, shape):
        self.__cuda_array_interface__ = {"data": (ptr, False), "shape": tuple(shape), "typestr": "<i2",
                                         "version": 3, "strides": None}


def stage_input_view(slot_id, b, t, d):
    """A bf16 [b, t, d] view of the slot's input buffer for a producer to
    write the next round's input into directly (an addition); the next
    submit then takes submit_staged_input_slot.  The view is valid until
    the slot's next prepare_* or staged submit."""
    ptr = c_vp()
    _lib.check(_L().swl_w_stage_input(int(slot_id), int(b), int(t), int(d), ctypes.byref(ptr)))
    raw = torch.as_tensor(_DeviceArray(ptr.value, (int(b), int(t), int(d))),
                          device=torch.device("cuda", _state["device"]))
    return raw.view(torch.bfloat16)


def prepare_token_ids_slot(slot_id, token_ids):
    if not isinstance(token_ids, torch.Tensor) or token_ids.dim() != 2:
        raise RuntimeError("token_ids must be 2D [B, T]")
    ids = _device_tensor(token_ids, "token_ids").to(torch.int64)
    b, t = ids.shape
    _lib.check(_L().swl_w_prepare_token_ids(int(slot_id), ids.data_ptr(), b, t, _stream()))


def get_embeddings_slot(slot_id, dtype):
    bx, tx, _ = _shape(slot_id)
    out = torch.empty(bx, tx, _state["hidden_dim"], dtype=dtype, device=torch.device("cuda", _state["device"]))
    _lib.check(_L().swl_w_copy_output(int(slot_id), out.data_ptr(), out.numel() * out.element_size(), _stream()))
    return out


def prepare_hidden_for_lm_head_slot(slot_id, hidden_states):
    if not isinstance(hidden_states, torch.Tensor) or hidden_states.dim() != 3:
        raise RuntimeError("hidden_states must be 3D [B, T, D]")
    h = _device_tensor(hidden_states, "hidden_states")
    b, t, d = h.shape
    _lib.check(_L().swl_w_prepare_hidden_lm(int(slot_id), h.data_ptr(), b, t, d, h.element_size(), _stream()))


def get_next_token_slot(slot_id):
    tok = c_i64(0)
    _lib.check(_L().swl_w_get_next_token(int(slot_id), ctypes.byref(tok), _stream()))
    return tok.value


def cleanup_worker_slots():
    _lib.check(_L().swl_w_cleanup())


# ------------------------------------------------ additions (no reference counterpart)
def set_gpu_ordered(enable=True, wait_outputs=True):
    """GPU-ordered slots: prepare_* stop waiting for their copy on the host
    and write the slot's next input sequence value on the stream instead;
    commands must then carry input_seq(slot_id).  wait_outputs: output reads
    first wait on the stream for the aggregator's output sequence word;
    without it they read the outputs at once, and the commands must carry
    out_host=True (the aggregator then finishes each round before
    signalling done)."""
    _lib.check(_L().swl_w_set_gpu_ordered(0 if not enable else (1 if wait_outputs else 2)))


def input_seq(slot_id):
    """Input sequence value written by the slot's last prepare_* call."""
    v = ctypes.c_uint64(0)
    _lib.check(_L().swl_w_input_seq(int(slot_id), ctypes.byref(v)))
    return v.value
