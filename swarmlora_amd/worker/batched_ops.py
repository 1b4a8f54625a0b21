"""Worker-side round helpers: attention over the paged KV cache and the
submit / signal / wait / read pattern of every aggregator round.

Mirrors src/worker/worker_sync.py: WorkerBatchedOps.batch_flash_attention
(:169-205) and BatchedAggregatorOps (:211-421), same method names and
arguments.  Attention is the libswl paged-attention kernel (RoPE, page
append and causal GQA attention in two launches) instead of vLLM's
rotary_embedding + flash_attn_with_kvcache.

One addition: with ``pooled_adapter`` set, the worker's adapter lives in the
aggregator's pool (ext_aggregator.register_adapter); commands carry
``x_key = pooled_adapter + 1`` and the aggregator adds the LoRA delta during
the scatter, so the worker skips its own delta products.
"""

import time
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch

from .. import ext_ipc_queue as extq
from .. import ext_unified_barrier as ub
from .. import ops
from .model_builder import OP_DOWN_PROJ, OP_EMBED, OP_GATE_UP_FUSED, OP_LM_HEAD, OP_O_PROJ, OP_QKV_FUSED
from .model_builder import SyncRemoteLoRALinear


class _NoStage:
    __slots__ = ()

    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_NO_STAGE = _NoStage()


class NullTimer:
    """Stage timer that times nothing (the unprofiled path)."""

    def stage(self, name):
        return _NO_STAGE


NULL_TIMER = NullTimer()


def _joined(parts):
    """The single [.., sum of widths] view that last-dim pieces of one buffer
    form (adjacent pieces, rows exactly their summed width), or None: lets a
    fused output and its fused delta be added in one launch."""
    p0 = parts[0]
    if p0 is None or p0.stride(-1) != 1:
        return None
    es = p0.element_size()
    total = sum(p.shape[-1] for p in parts if p is not None)
    off = p0.data_ptr()
    base = p0.untyped_storage().data_ptr()
    for p in parts:
        if (p is None or p.shape[:-1] != p0.shape[:-1] or p.stride() != p0.stride() or p.data_ptr() != off or
                p.untyped_storage().data_ptr() != base):
            return None
        off += p.shape[-1] * es
    for i in range(p0.dim() - 1):
        if p0.shape[i] > 1 and p0.stride(i) != total * p0.shape[i + 1:-1].numel():
            return None
    return p0.as_strided((*p0.shape[:-1], total), p0.stride())


def _add_deltas(raw, deltas):
    """raw[i] += deltas[i] (bf16, in place on the worker-owned output copy),
    one launch when both sides are pieces of one buffer each."""
    if all(d is None for d in deltas):
        return
    if all(d is not None for d in deltas):
        jr, jd = _joined(raw), _joined(deltas)
        if jr is not None and jd is not None and jr.shape == jd.shape:
            jr.add_(jd)
            return
    for r, d in zip(raw, deltas):
        if d is not None:
            r.add_(d)


@dataclass
class SlotState:
    """Per-request state of an active slot (worker_sync.py:100-118)."""
    slot_id: int
    input_ids: torch.Tensor
    generated_tokens: List[int] = field(default_factory=list)
    hidden: Optional[torch.Tensor] = None
    residual: Optional[torch.Tensor] = None
    mlp_residual: Optional[torch.Tensor] = None
    prefill_chunks: Optional[list] = None
    first_token_time: Optional[float] = None


class WorkerBatchedOps:
    @staticmethod
    def batch_flash_attention(slot_ids: list, qkv_results: dict, paged_kv, cos_sin_cache: torch.Tensor,
                              layer_idx: int, num_heads: int, num_kv_heads: int, head_dim: int,
                              attn_meta: dict = None, out: Optional[Dict[int, torch.Tensor]] = None
                              ) -> Dict[int, torch.Tensor]:
        """RoPE at attn_meta['positions'], append k/v at cache_seqlens, causal
        GQA attention over the pages; returns {slot: [1, q_len, hidden]}.
        q/k/v may be views of the fused QKV output (read in place).  out (an
        addition): {slot: [1, q_len, hidden] bf16} to write a lone slot's
        result into (a staged slot input buffer)."""
        q_len = attn_meta["bufs_q"].shape[1]
        n = len(slot_ids)

        def gather(j, heads):
            parts = [qkv_results[s][j].reshape(1, q_len, heads, head_dim) for s in slot_ids]
            return parts[0] if n == 1 else torch.cat(parts, 0)

        q = gather(0, num_heads)
        k = gather(1, num_kv_heads)
        v = gather(2, num_kv_heads)
        dst = out.get(slot_ids[0]) if out is not None and n == 1 else None
        out = ops.paged_attention(q, k, v, paged_kv.key_caches[layer_idx], paged_kv.value_caches[layer_idx],
                                  attn_meta["block_tables"], attn_meta["cache_seqlens"], attn_meta["positions"],
                                  cos_sin_cache, 1.0 / (head_dim ** 0.5), out=dst)
        return {sid: out[i:i + 1] for i, sid in enumerate(slot_ids)}


class BatchedAggregatorOps:
    """submit -> signal_ready -> (local LoRA delta) -> wait epoch -> read."""

    def __init__(self, slot_manager, worker_id: int, dtype_code: int, pooled_adapter: Optional[int] = None,
                 gpu_ordered=False):
        self.slot_manager = slot_manager
        self.worker_id = worker_id
        # gpu_ordered (an addition): slot copies are ordered against the
        # aggregator's rounds on the GPU (sequence words in the slot buffer)
        # instead of by host waits.  True: inputs and outputs, barrier_sync
        # then returns once the round is launched, not finished; "inputs":
        # the input copy only (no host wait before the submit), the outputs
        # read once the round has finished, as in the reference
        if gpu_ordered not in (False, True, "inputs"):
            raise ValueError("gpu_ordered must be False, True or 'inputs'")
        self.gpu_ordered = gpu_ordered
        self._out_host = gpu_ordered == "inputs"
        if gpu_ordered:
            ub.set_gpu_ordered(True, wait_outputs=not self._out_host)
        # slots whose input buffer already holds the next round's input (a
        # fused read staged it there): their next submit copies nothing
        self._staged = set()
        self.dtype_code = dtype_code
        self.dtype = torch.bfloat16 if dtype_code == 15 else torch.float16
        self.hidden_dim = slot_manager.base_client.hidden_dim
        self.pooled_adapter = pooled_adapter
        self._x_key = 0 if pooled_adapter is None else int(pooled_adapter) + 1
        # stage timer of WorkerEngine's profiled path (times nothing otherwise)
        self.timer = NULL_TIMER

    def barrier_sync(self, epoch: int):
        extq.wait_for_epoch(epoch)

    def _get_outputs_all(self, slots, dims):
        slot_id, state = next(iter(slots.items()))
        with self.timer.stage("scatter"):
            return {slot_id: ub.get_outputs_slot(slot_id, dims, state.hidden)}

    def _fused_read(self, slots, dims, delta=None, residual=None):
        """The slot's output with the caller's adds in the same launch
        (ub.read_outputs_slot), or None where the operands do not fit it
        (then the caller copies and adds on its own)."""
        slot_id, state = next(iter(slots.items()))
        tmpl = state.hidden
        if tmpl is None or tmpl.dtype != torch.bfloat16 or len(slots) != 1:
            return None
        for t in (delta, residual):
            if t is not None and (t.dtype != torch.bfloat16 or not t.is_contiguous() or t.shape[-1] != sum(dims)
                                  or t.dim() != 3):
                return None
        with self.timer.stage("scatter"):
            return ub.read_outputs_slot(slot_id, dims, tmpl, delta, residual)

    def _one_bf16_slot(self, slots):
        """The (slot, state) of a single-slot worker whose rows are bf16, or
        None (the fused reads below serve that case)."""
        if len(slots) != 1:
            return None
        sid, state = next(iter(slots.items()))
        if state.hidden is None or state.hidden.dtype != torch.bfloat16:
            return None
        return sid, state

    @staticmethod
    def _fits(t, d):
        return t is None or (t.dtype == torch.bfloat16 and t.is_contiguous() and t.dim() == 3 and t.shape[-1] == d
                             and t.data_ptr() % 16 == 0)

    def o_proj_get_norm_all(self, slots, layer_idx: int, deltas, out_dim: int, weight, eps: float,
                            stage: bool = False) -> bool:
        """o_proj_get_all and the post-attention norm the caller runs next, in
        one launch (an addition): state.mlp_residual = residual + (o + delta),
        state.hidden = its RMSNorm; False (nothing done) when the operands do
        not fit, then the caller takes the separate steps."""
        one = self._one_bf16_slot(slots)
        if one is None or out_dim % 8:
            return False
        sid, state = one
        d = deltas.get(sid)
        if not (self._fits(d, out_dim) and self._fits(state.residual, out_dim)):
            return False
        with self.timer.stage("scatter"):
            state.mlp_residual, state.hidden = ub.read_outputs_norm_slot(sid, out_dim, state.hidden, d,
                                                                         state.residual, weight, eps, stage)
        if stage:
            self._staged.add(sid)
        return True

    def down_proj_get_norm_all(self, slots, layer_idx: int, deltas, out_dim: int, weight, eps: float,
                               stage: bool = False) -> bool:
        """down_proj_get_all and the next norm (the next layer's input norm or
        the final norm) in one launch (an addition): state.residual =
        mlp_residual + (down + delta), state.hidden = its RMSNorm."""
        one = self._one_bf16_slot(slots)
        if one is None or out_dim % 8:
            return False
        sid, state = one
        d = deltas.get(sid)
        if not (self._fits(d, out_dim) and self._fits(state.mlp_residual, out_dim)):
            return False
        with self.timer.stage("scatter"):
            state.residual, state.hidden = ub.read_outputs_norm_slot(sid, out_dim, state.hidden, d,
                                                                     state.mlp_residual, weight, eps, stage)
        if stage:
            self._staged.add(sid)
        return True

    def gate_up_get_act_all(self, slots, layer_idx: int, deltas, dims: List[int], stage: bool = False):
        """gate_up_get_all and the SiLU*up the caller runs next, in one launch
        (an addition): {slot: act [B, T, inter]}, or None when the operands
        do not fit (then the caller takes the separate steps)."""
        one = self._one_bf16_slot(slots)
        if one is None or len(dims) != 2 or dims[0] != dims[1] or dims[0] % 8:
            return None
        sid, state = one
        d = list(deltas.get(sid, (None, None)))
        if all(x is None for x in d):
            jd = None
        elif any(x is None for x in d):
            return None
        else:
            jd = _joined(d)
            if jd is None or not self._fits(jd, 2 * dims[0]):
                return None
        with self.timer.stage("scatter"):
            act = ub.read_outputs_silu_slot(sid, dims[0], state.hidden, jd, stage)
        if stage:
            self._staged.add(sid)
        return {sid: act}

    def stage_attn_outputs(self, slots, q_len: int, width: int):
        """{slot: [1, q_len, width] view of the slot's input buffer} for the
        attention to write the O round's input into (an addition), so that
        round's submit copies nothing; None when the slot's rows are not
        bf16 or do not fit the buffer."""
        one = self._one_bf16_slot(slots)
        if one is None or width % 8:
            return None
        sid, state = one
        try:
            view = ub.stage_input_view(sid, 1, q_len, width)
        except RuntimeError:
            return None
        self._staged.add(sid)
        return {sid: view}

    def _fused_join(self, slots, deltas, dims, n):
        """qkv / gate_up read: the fused output plus its fused delta in one
        launch when the per-block deltas are pieces of one buffer."""
        sid = next(iter(slots))
        d = list(deltas.get(sid, (None,) * n))
        if all(x is None for x in d):
            jd = None
        elif any(x is None for x in d):
            return None
        else:
            jd = _joined(d)
            if jd is None:
                return None
        got = self._fused_read(slots, dims, jd, None)
        return None if got is None else {sid: tuple(got)}

    def _seq(self, slot_id):
        return ub.input_seq(slot_id) if self.gpu_ordered else 0

    def _submit(self, op, layer_idx, slot_id, x):
        b, t, d = x.shape
        with self.timer.stage("gather"):
            if slot_id in self._staged:
                self._staged.discard(slot_id)
                ub.submit_staged_input_slot(slot_id, x)
            else:
                ub.prepare_input_slot(slot_id, op, x)
            extq.submit_slot_command(op, layer_idx, slot_id, self.worker_id, b, t, d, self._x_key, 0, 0, 0, 0,
                                     in_seq=self._seq(slot_id), out_host=self._out_host)
            extq.slot_signal_ready(slot_id)

    # ---------------------------------------------------------------- embed
    def embed_submit_all(self, slots) -> int:
        self._staged.clear()  # nothing staged crosses a token boundary
        epoch = extq.get_barrier_done_epoch()
        slot_id, state = next(iter(slots.items()))
        ub.prepare_token_ids_slot(slot_id, state.input_ids)
        b, t = state.input_ids.shape
        extq.submit_slot_command(OP_EMBED, 0, slot_id, self.worker_id, b, t, self.hidden_dim, 0, 0, 0, 0, 0,
                                 in_seq=self._seq(slot_id), out_host=self._out_host)
        extq.slot_signal_ready(slot_id)
        return epoch

    def embed_get_all(self, slots):
        slot_id, state = next(iter(slots.items()))
        state.hidden = ub.get_embeddings_slot(slot_id, self.dtype)

    # ------------------------------------------------------------------ QKV
    def qkv_submit_all(self, slots, layer_idx: int, fused_qkv_modules: List):
        epoch = extq.get_barrier_done_epoch()
        slot_id, state = next(iter(slots.items()))
        self._submit(OP_QKV_FUSED, layer_idx, slot_id, state.hidden)
        fq = fused_qkv_modules[layer_idx]
        with self.timer.stage("lora"):
            if self.pooled_adapter is None and fq.fused_lora is not None and fq.fused_lora.has_lora:
                deltas = {slot_id: fq.fused_lora(state.hidden)}
            else:
                deltas = {slot_id: (None, None, None)}
        return epoch, deltas

    def qkv_get_all(self, slots, layer_idx: int, deltas, dims: List[int]):
        fused = self._fused_join(slots, deltas, dims, 3)
        if fused is not None:
            return fused
        raw = self._get_outputs_all(slots, dims)
        res = {}
        with self.timer.stage("lora"):
            for sid in slots:
                # q + dq, k + dk, v + dv (bf16) on the fresh output copy
                _add_deltas(raw[sid], list(deltas.get(sid, (None, None, None))))
                res[sid] = tuple(raw[sid])
        return res

    # -------------------------------------------------------------------- O
    def o_proj_submit_all(self, slots, layer_idx: int, attn_outputs, o_proj_modules: List):
        epoch = extq.get_barrier_done_epoch()
        slot_id, state = next(iter(slots.items()))
        x = attn_outputs[slot_id]
        self._submit(OP_O_PROJ, layer_idx, slot_id, x)
        o = o_proj_modules[layer_idx]
        use = self.pooled_adapter is None and isinstance(o, SyncRemoteLoRALinear)
        with self.timer.stage("lora"):
            return epoch, {slot_id: o.delta(x) if use else None}

    def o_proj_get_all(self, slots, layer_idx: int, deltas, out_dim: int):
        sid, state = next(iter(slots.items()))
        got = self._fused_read(slots, [out_dim], deltas.get(sid), state.residual)
        if got is not None:  # residual + (o + delta), one launch
            state.hidden = got[0]
            return
        raw = self._get_outputs_all(slots, [out_dim])
        with self.timer.stage("lora"):
            for sid, state in slots.items():
                r = raw[sid][0]
                d = deltas.get(sid)
                if d is not None:
                    r = r + d
                state.hidden = state.residual + r

    # -------------------------------------------------------------- Gate+Up
    def gate_up_submit_all(self, slots, layer_idx: int, fused_gate_up_modules: List):
        epoch = extq.get_barrier_done_epoch()
        slot_id, state = next(iter(slots.items()))
        self._submit(OP_GATE_UP_FUSED, layer_idx, slot_id, state.hidden)
        fg = fused_gate_up_modules[layer_idx]
        with self.timer.stage("lora"):
            if self.pooled_adapter is None and fg.fused_lora is not None and fg.fused_lora.has_lora:
                deltas = {slot_id: fg.fused_lora(state.hidden)}
            else:
                deltas = {slot_id: (None, None)}
        return epoch, deltas

    def gate_up_get_all(self, slots, layer_idx: int, deltas, dims: List[int]):
        # g and u are the two halves of the freshly copied output; the deltas
        # are added in place (the values of g + dg, u + du) so the pair stays
        # one [.., 2 * inter] buffer that the SiLU*up kernel reads directly
        fused = self._fused_join(slots, deltas, dims, 2)
        if fused is not None:
            return fused
        raw = self._get_outputs_all(slots, dims)
        res = {}
        with self.timer.stage("lora"):
            for sid in slots:
                _add_deltas(raw[sid], list(deltas.get(sid, (None, None))))
                res[sid] = tuple(raw[sid])
        return res

    # ----------------------------------------------------------------- Down
    def down_proj_submit_all(self, slots, layer_idx: int, mlp_intermediates, down_proj_modules: List):
        epoch = extq.get_barrier_done_epoch()
        slot_id, state = next(iter(slots.items()))
        x = mlp_intermediates[slot_id]
        self._submit(OP_DOWN_PROJ, layer_idx, slot_id, x)
        dp = down_proj_modules[layer_idx]
        use = self.pooled_adapter is None and isinstance(dp, SyncRemoteLoRALinear)
        with self.timer.stage("lora"):
            return epoch, {slot_id: dp.delta(x) if use else None}

    def down_proj_get_all(self, slots, layer_idx: int, deltas, out_dim: int):
        sid, state = next(iter(slots.items()))
        got = self._fused_read(slots, [out_dim], deltas.get(sid), state.mlp_residual)
        if got is not None:  # mlp_residual + (down + delta), one launch
            state.hidden = got[0]
            return
        raw = self._get_outputs_all(slots, [out_dim])
        with self.timer.stage("lora"):
            for sid, state in slots.items():
                r = raw[sid][0]
                d = deltas.get(sid)
                if d is not None:
                    r = r + d
                state.hidden = state.mlp_residual + r

    # -------------------------------------------------------------- LM head
    def lm_head_submit_all(self, slots) -> int:
        epoch = extq.get_barrier_done_epoch()
        slot_id, state = next(iter(slots.items()))
        ub.prepare_hidden_for_lm_head_slot(slot_id, state.hidden)
        b, t, d = state.hidden.shape
        extq.submit_slot_command(OP_LM_HEAD, 0, slot_id, self.worker_id, b, t, d, 0, 0, 0, 0, 0,
                                 in_seq=self._seq(slot_id), out_host=self._out_host)
        extq.slot_signal_ready(slot_id)
        return epoch

    def lm_head_get_all(self, slots):
        for slot_id, state in slots.items():
            tok = ub.get_next_token_slot(slot_id)
            if state.prefill_chunks:
                state.input_ids = state.prefill_chunks.pop(0)
                if not state.prefill_chunks:
                    state.prefill_chunks = None
            else:
                if state.first_token_time is None:
                    state.first_token_time = time.perf_counter()
                state.generated_tokens.append(tok)
                state.input_ids = torch.tensor([[tok]], device=state.input_ids.device)
