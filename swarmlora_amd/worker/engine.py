"""Per-token driver of a worker: the 130-round sequence of one decode step.

Follows BatchedInferenceEngine._generate_one_token_all
(src/worker/worker_sync.py:1274-1425): eviction check, KV page reservation,
attention metadata per q_len, the embed round, per layer RMSNorm -> QKV round
-> attention -> O round -> RMSNorm -> Gate+Up round -> SiLU*up -> Down round,
sequence lengths advanced after all layers, final norm, the LM-head round.
The HTTP/request-queue shell around it (FaaSWorker) is not part of this
package.  RMSNorm and SiLU*up are torch elementwise ops on the worker's GPU.
"""

from collections import defaultdict
from dataclasses import dataclass
from typing import Callable, Dict, List, Optional

import torch
import torch.nn.functional as F

from .. import ext_ipc_queue as extq
from .batched_ops import BatchedAggregatorOps, SlotState, WorkerBatchedOps


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """LlamaRMSNorm: fp32 variance, x * rsqrt(var + eps) cast back, * weight."""
    xf = x.float()
    var = xf.pow(2).mean(-1, keepdim=True)
    return weight * (xf * torch.rsqrt(var + eps)).to(x.dtype)


@dataclass
class LayerModules:
    input_norm: torch.Tensor
    post_norm: torch.Tensor
    fused_qkv: object      # SyncFusedQKV
    o_proj: object         # SyncRemoteLinear / SyncRemoteLoRALinear
    fused_gate_up: object  # SyncFusedGateUp
    down_proj: object


class WorkerEngine:
    def __init__(self, layers: List[LayerModules], final_norm: torch.Tensor, eps: float, num_heads: int,
                 num_kv_heads: int, head_dim: int, paged_kv, cos_sin_cache: torch.Tensor,
                 ops: BatchedAggregatorOps, on_evicted: Optional[Callable[[int, SlotState], None]] = None):
        self.layers = layers
        self.final_norm = final_norm
        self.eps = eps
        self.num_heads, self.num_kv_heads, self.head_dim = num_heads, num_kv_heads, head_dim
        self.hidden = num_heads * head_dim
        self.kv = paged_kv
        self.cos_sin = cos_sin_cache
        self.ops = ops
        self.on_evicted = on_evicted
        self.qkv_dims = [self.hidden, num_kv_heads * head_dim, num_kv_heads * head_dim]

    def generate_one_token_all(self, slots: Dict[int, SlotState], record: Optional[list] = None):
        for sid in list(slots):
            if extq.is_slot_evicted(sid):
                extq.clear_evicted_slot(sid)
                st = slots.pop(sid)
                if self.on_evicted:
                    self.on_evicted(sid, st)
        if not slots:
            return
        for sid, st in list(slots.items()):
            self.kv.ensure_blocks_for_length(sid, self.kv.slot_seq_lens.get(sid, 0) + st.input_ids.size(1))
        groups = defaultdict(list)
        for sid, st in slots.items():
            groups[st.input_ids.size(1)].append(sid)
        dev = self.cos_sin.device
        metas = {}
        for q_len, sids in groups.items():
            seqlens = self.kv.get_seq_lens_tensor(sids)
            pos = (seqlens.long().unsqueeze(1) + torch.arange(q_len, device=dev).unsqueeze(0)).reshape(-1)
            metas[q_len] = {"cache_seqlens": seqlens, "block_tables": self.kv.get_block_table_tensor(sids),
                            "positions": pos, "bufs_q": torch.empty(len(sids), q_len, 0, device=dev)}

        ops = self.ops
        ops.barrier_sync(ops.embed_submit_all(slots))
        ops.embed_get_all(slots)
        qkv_mods = [l.fused_qkv for l in self.layers]
        o_mods = [l.o_proj for l in self.layers]
        gu_mods = [l.fused_gate_up for l in self.layers]
        dn_mods = [l.down_proj for l in self.layers]
        for li, layer in enumerate(self.layers):
            for st in slots.values():
                st.residual = st.hidden
                st.hidden = rms_norm(st.hidden, layer.input_norm, self.eps)
            epoch, deltas = ops.qkv_submit_all(slots, li, qkv_mods)
            ops.barrier_sync(epoch)
            qkv = ops.qkv_get_all(slots, li, deltas, layer.fused_qkv.dims)
            attn = {}
            for q_len, sids in groups.items():
                attn.update(WorkerBatchedOps.batch_flash_attention(sids, qkv, self.kv, self.cos_sin, li,
                                                                   self.num_heads, self.num_kv_heads,
                                                                   self.head_dim, metas[q_len]))
            epoch, deltas = ops.o_proj_submit_all(slots, li, attn, o_mods)
            ops.barrier_sync(epoch)
            ops.o_proj_get_all(slots, li, deltas, self.hidden)
            for st in slots.values():
                st.mlp_residual = st.hidden
                st.hidden = rms_norm(st.hidden, layer.post_norm, self.eps)
            epoch, deltas = ops.gate_up_submit_all(slots, li, gu_mods)
            ops.barrier_sync(epoch)
            gu = ops.gate_up_get_all(slots, li, deltas, layer.fused_gate_up.dims)
            mlp = {sid: F.silu(g) * u for sid, (g, u) in gu.items()}
            epoch, deltas = ops.down_proj_submit_all(slots, li, mlp, dn_mods)
            ops.barrier_sync(epoch)
            ops.down_proj_get_all(slots, li, deltas, self.hidden)
        sids = list(slots)
        self.kv.advance_seq_lens_by(sids, [slots[s].input_ids.size(1) for s in sids])
        for st in slots.values():
            st.hidden = rms_norm(st.hidden, self.final_norm, self.eps)
            if st.prefill_chunks:
                st.hidden = st.hidden[:, -1:, :]
        if record is not None:
            record.append({sid: (slots[sid].input_ids.clone(), slots[sid].hidden.clone()) for sid in sids})
        ops.barrier_sync(ops.lm_head_submit_all(slots))
        ops.lm_head_get_all(slots)
