"""Per-token driver of a worker: the 130-round sequence of one decode step.

Follows BatchedInferenceEngine._generate_one_token_all
(src/worker/worker_sync.py:1274-1425): eviction check, KV page reservation,
attention metadata per q_len, the embed round, per layer RMSNorm -> QKV round
-> attention -> O round -> RMSNorm -> Gate+Up round -> SiLU*up -> Down round,
sequence lengths advanced after all layers, final norm, the LM-head round.
The HTTP/request-queue shell around it (FaaSWorker) is not part of this
package.  RMSNorm and SiLU*up run as libswl row kernels on the worker's GPU.

With PROFILE_LAYERS=1 in the environment (or profile=True) every token is
timed by stage, with a device synchronisation around each stage, and one
line per decode token is printed in the reference's format
(worker_sync.py:1427-1782, the line at :1774-1777):
``[LAYER_PROFILE] worker=W token=N gather_us=.. scatter_us=.. compute_us=..
wall_us=.. ipc_pct=..`` followed by this build's finer split (gemm_us: the
wait for the aggregator's round, lora_us: the worker's own LoRA products and
adds, attn_us: norms, attention and SiLU*up).  gather is input copy +
command submit + ready signal, scatter is the output copy; compute_us is
wall_us minus the two.
"""

import os
import time
from collections import defaultdict
from dataclasses import dataclass
from typing import Callable, Dict, List, Optional

import torch

from .. import ext_ipc_queue as extq
from .. import ops
from .batched_ops import NULL_TIMER, BatchedAggregatorOps, SlotState, WorkerBatchedOps


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """LlamaRMSNorm (fp32 variance, x * rsqrt(var + eps) cast back, * weight)
    on the libswl row kernel."""
    return ops.rms_norm(x.contiguous(), weight, eps)


def silu_mul(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """F.silu(g) * u on the libswl row kernel; g and u are read in place when
    they are the two halves of one fused Gate+Up output."""
    inter = g.shape[-1]
    es = g.element_size()
    if (u.shape == g.shape and g.stride() == u.stride() and g.stride(-1) == 1 and
            g.untyped_storage().data_ptr() == u.untyped_storage().data_ptr() and
            u.data_ptr() == g.data_ptr() + inter * es and
            all(g.stride(i) == 2 * inter * g.shape[i + 1:-1].numel() for i in range(g.dim() - 1))):
        gu = g.as_strided((*g.shape[:-1], 2 * inter), g.stride())
    else:
        gu = torch.cat([g, u], -1)
    return ops.silu_mul(gu, inter)


class StageTimer:
    """Accumulates per-stage wall time of one token, synchronising the device
    around each stage (the profiled path of worker_sync.py:1427-1782)."""

    STAGES = ("gather", "gemm", "scatter", "lora", "attn")

    def __init__(self):
        self.token = 0
        self.records: List[dict] = []
        self.reset()

    def reset(self):
        self.us = dict.fromkeys(self.STAGES, 0.0)
        torch.cuda.synchronize()
        self.t_start = time.perf_counter()

    def stage(self, name):
        return _Stage(self, name)

    def finish(self, worker_id: int, batch: int, log: bool = True) -> dict:
        torch.cuda.synchronize()
        wall = (time.perf_counter() - self.t_start) * 1e6
        self.token += 1
        ipc = self.us["gather"] + self.us["scatter"]
        rec = {"batch": batch, "token": self.token, "gather_us": self.us["gather"],
               "scatter_us": self.us["scatter"], "compute_us": wall - ipc, "wall_us": wall,
               "gemm_us": self.us["gemm"], "lora_us": self.us["lora"], "attn_us": self.us["attn"]}
        self.records.append(rec)
        if log:
            print(f"[LAYER_PROFILE] worker={worker_id} token={self.token} "
                  f"gather_us={rec['gather_us']:.0f} scatter_us={rec['scatter_us']:.0f} "
                  f"compute_us={rec['compute_us']:.0f} wall_us={wall:.0f} "
                  f"ipc_pct={(ipc / wall * 100 if wall > 0 else 0):.1f} "
                  f"gemm_us={rec['gemm_us']:.0f} lora_us={rec['lora_us']:.0f} attn_us={rec['attn_us']:.0f}",
                  flush=True)
        return rec


class _Stage:
    __slots__ = ("t", "name", "t0")

    def __init__(self, timer, name):
        self.t, self.name = timer, name

    def __enter__(self):
        torch.cuda.synchronize()
        self.t0 = time.perf_counter()

    def __exit__(self, *exc):
        torch.cuda.synchronize()
        self.t.us[self.name] += (time.perf_counter() - self.t0) * 1e6
        return False


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
                 ops: BatchedAggregatorOps, on_evicted: Optional[Callable[[int, SlotState], None]] = None,
                 profile: Optional[bool] = None):
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
        if profile is None:
            profile = os.environ.get("PROFILE_LAYERS") == "1"
        self.profiler = StageTimer() if profile else None

    def generate_one_token_all(self, slots: Dict[int, SlotState], record: Optional[list] = None):
        prof = self.profiler
        if prof is not None:
            prof.reset()
        tm = prof if prof is not None else NULL_TIMER
        for sid in list(slots):
            if extq.is_slot_evicted(sid):
                extq.clear_evicted_slot(sid)
                st = slots.pop(sid)
                if self.on_evicted:
                    self.on_evicted(sid, st)
        if not slots:
            return
        has_prefill = any(st.input_ids.size(1) > 1 or st.prefill_chunks for st in slots.values())
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
        ops.timer = tm
        with tm.stage("gather"):
            epoch = ops.embed_submit_all(slots)
        with tm.stage("gemm"):
            ops.barrier_sync(epoch)
        with tm.stage("scatter"):
            ops.embed_get_all(slots)
        qkv_mods = [l.fused_qkv for l in self.layers]
        o_mods = [l.o_proj for l in self.layers]
        gu_mods = [l.fused_gate_up for l in self.layers]
        dn_mods = [l.down_proj for l in self.layers]
        # The O and Down outputs are read together with the norm that follows
        # each (and the Gate+Up output with SiLU*up) where the operands allow,
        # one launch instead of three; `normed` says the Down read already
        # produced the next layer's normalised input (or the final norm).
        normed = False
        for li, layer in enumerate(self.layers):
            with tm.stage("attn"):
                if not normed:
                    for st in slots.values():
                        st.residual = st.hidden
                        st.hidden = rms_norm(st.hidden, layer.input_norm, self.eps)
            epoch, deltas = ops.qkv_submit_all(slots, li, qkv_mods)
            with tm.stage("gemm"):
                ops.barrier_sync(epoch)
            qkv = ops.qkv_get_all(slots, li, deltas, layer.fused_qkv.dims)
            with tm.stage("attn"):
                attn = {}
                # a lone slot's attention writes straight into its input
                # buffer: the O round's submit then copies nothing
                staged = (ops.stage_attn_outputs(slots, next(iter(groups)), self.num_heads * self.head_dim)
                          if len(groups) == 1 else None)
                for q_len, sids in groups.items():
                    attn.update(WorkerBatchedOps.batch_flash_attention(sids, qkv, self.kv, self.cos_sin, li,
                                                                       self.num_heads, self.num_kv_heads,
                                                                       self.head_dim, metas[q_len], out=staged))
            epoch, deltas = ops.o_proj_submit_all(slots, li, attn, o_mods)
            with tm.stage("gemm"):
                ops.barrier_sync(epoch)
            # stage=True: the fused read also writes the next round's input
            # into the slot's input buffer, so that round's submit copies
            # nothing
            if not ops.o_proj_get_norm_all(slots, li, deltas, self.hidden, layer.post_norm, self.eps, stage=True):
                ops.o_proj_get_all(slots, li, deltas, self.hidden)
                with tm.stage("attn"):
                    for st in slots.values():
                        st.mlp_residual = st.hidden
                        st.hidden = rms_norm(st.hidden, layer.post_norm, self.eps)
            epoch, deltas = ops.gate_up_submit_all(slots, li, gu_mods)
            with tm.stage("gemm"):
                ops.barrier_sync(epoch)
            mlp = ops.gate_up_get_act_all(slots, li, deltas, layer.fused_gate_up.dims, stage=True)
            if mlp is None:
                gu = ops.gate_up_get_all(slots, li, deltas, layer.fused_gate_up.dims)
                with tm.stage("attn"):
                    mlp = {sid: silu_mul(g, u) for sid, (g, u) in gu.items()}
            epoch, deltas = ops.down_proj_submit_all(slots, li, mlp, dn_mods)
            with tm.stage("gemm"):
                ops.barrier_sync(epoch)
            nxt = self.layers[li + 1].input_norm if li + 1 < len(self.layers) else self.final_norm
            normed = ops.down_proj_get_norm_all(slots, li, deltas, self.hidden, nxt, self.eps,
                                                stage=li + 1 < len(self.layers))
            if not normed:
                ops.down_proj_get_all(slots, li, deltas, self.hidden)
        sids = list(slots)
        self.kv.advance_seq_lens_by(sids, [slots[s].input_ids.size(1) for s in sids])
        with tm.stage("attn"):
            for st in slots.values():
                if not normed:
                    st.hidden = rms_norm(st.hidden, self.final_norm, self.eps)
                if st.prefill_chunks:
                    st.hidden = st.hidden[:, -1:, :]
        if record is not None:
            record.append({sid: (slots[sid].input_ids.clone(), slots[sid].hidden.clone()) for sid in sids})
        with tm.stage("gather"):
            epoch = ops.lm_head_submit_all(slots)
        with tm.stage("gemm"):
            ops.barrier_sync(epoch)
        with tm.stage("scatter"):
            ops.lm_head_get_all(slots)
        ops.timer = NULL_TIMER
        if prof is not None:
            prof.finish(ops.worker_id, len(slots), log=not has_prefill)
