"""Adapter lifecycle: hot swap of a worker's LoRA modules, and the HBM pool
the aggregator's pooled rounds read.

AdapterManager mirrors src/worker/adapter_manager.py:13-280: the same
constructor, getters and swap_adapter() result dictionary.  A swap with an
unchanged rank writes the new weights into the existing tensors (the
reference's in-place fast path, :107-195); a rank change rebuilds the fused
modules (:212-280).  The model may be shaped like the reference's hollow
model (model.model.layers[i].self_attn._fused_qkv / .o_proj,
.mlp._fused_gate_up / .down_proj) or be this package's WorkerEngine /
list of LayerModules.

AdapterPool holds whole adapters resident in HBM for the aggregator's
pooled LoRA (ext_aggregator.register_adapter, one entry per (adapter, layer,
fused projection)) -- the config-5 serving mode where many adapters stay on
the GPU and each slot names one.  Its swap keeps the device pointers when the
rank is unchanged: the round kernels plan from the pointers and read the
scale from the device table, so rounds captured in a HIP graph keep working
after an in-place swap.  A swap that changes the rank registers new tensors;
graphs captured before it must be captured again.
"""

import threading
import time
import traceback
from typing import Dict, Iterator, List, Sequence, Tuple

import torch

from .model_builder import FusedLoRA, SyncRemoteLoRALinear, load_lora_fast

QKV_NAMES = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj")
GATE_UP_NAMES = ("mlp.gate_proj", "mlp.up_proj")
O_NAME = "self_attn.o_proj"
DOWN_NAME = "mlp.down_proj"


def _scaling(config: dict) -> float:
    return config.get("lora_alpha", config["r"]) / config["r"]


def _layer_slots(model) -> Iterator[Tuple[int, object, object, object, object, object, object]]:
    """(layer index, qkv holder, gate/up holder, o_proj owner, o_proj, down owner,
    down_proj) for each decoder layer; holders carry .fused_lora, owners are
    the objects whose o_proj / down_proj attribute may be replaced."""
    layers = None
    inner = getattr(model, "model", None)
    if inner is not None and hasattr(inner, "layers"):
        for i, layer in enumerate(inner.layers):
            attn, mlp = layer.self_attn, layer.mlp
            yield (i, getattr(attn, "_fused_qkv", None), getattr(mlp, "_fused_gate_up", None),
                   attn, getattr(attn, "o_proj", None), mlp, getattr(mlp, "down_proj", None))
        return
    layers = model.layers if hasattr(model, "layers") else model
    for i, layer in enumerate(layers):
        yield (i, getattr(layer, "fused_qkv", None), getattr(layer, "fused_gate_up", None),
               layer, getattr(layer, "o_proj", None), layer, getattr(layer, "down_proj", None))


class AdapterManager:
    """One worker's adapter state with a thread-safe hot swap."""

    def __init__(self, worker_id: int, device, dtype: torch.dtype, info: dict):
        self.worker_id = worker_id
        self.device = device
        self.dtype = dtype
        self.info = info
        self.current_adapter_id = None
        self.current_rank = 0
        self.current_config = None
        self._swap_lock = threading.Lock()
        self._is_swapping = threading.Event()

    def get_current_adapter(self):
        with self._swap_lock:
            return self.current_adapter_id

    def is_swapping(self) -> bool:
        return self._is_swapping.is_set()

    def set_adapter(self, adapter_id: str, rank: int, config: dict):
        """Record the adapter the model was built with."""
        with self._swap_lock:
            self.current_adapter_id = adapter_id
            self.current_rank = rank
            self.current_config = config

    def swap_adapter(self, new_adapter_id: str, model) -> dict:
        """Load adapter directory `new_adapter_id` (PEFT safetensors) and make
        the model's LoRA modules use it.  Returns timings and what changed,
        or {'success': False, 'error': ...} with the model unchanged when the
        load fails."""
        t0 = time.perf_counter()
        with self._swap_lock:
            self._is_swapping.set()
            try:
                old_id, old_rank = self.current_adapter_id, self.current_rank
                t_load = time.perf_counter()
                layers, config = load_lora_fast(new_adapter_id, self.device, self.dtype)
                new_rank = config["r"]
                t_loaded = time.perf_counter()
                rank_changed = old_rank not in (0, new_rank)
                t_upd = time.perf_counter()
                if rank_changed:
                    self._recreate_lora_modules(model, layers, config)
                else:
                    self._update_lora_weights(model, layers, config)
                if torch.cuda.is_available() and str(self.device).startswith("cuda"):
                    torch.cuda.synchronize()
                t_done = time.perf_counter()
                self.current_adapter_id, self.current_rank, self.current_config = new_adapter_id, new_rank, config
                return {
                    "success": True,
                    "old_adapter": old_id,
                    "new_adapter": new_adapter_id,
                    "old_rank": old_rank,
                    "new_rank": new_rank,
                    "rank_changed": rank_changed,
                    "load_time_ms": round((t_loaded - t_load) * 1000, 2),
                    "update_time_ms": round((t_done - t_upd) * 1000, 2),
                    "total_time_ms": round((time.perf_counter() - t0) * 1000, 2),
                }
            except Exception as e:  # the reference reports instead of raising
                traceback.print_exc()
                return {"success": False, "error": str(e)}
            finally:
                self._is_swapping.clear()

    # ------------------------------------------------------------ same rank
    def _update_lora_weights(self, model, layers: dict, config: dict):
        s = _scaling(config)
        for li, qkv, gu, _, o_proj, _, down in _layer_slots(model):
            if qkv is not None and getattr(qkv, "fused_lora", None) is not None:
                self._update_fused_lora(qkv.fused_lora, QKV_NAMES, li, layers, s)
            if gu is not None and getattr(gu, "fused_lora", None) is not None:
                self._update_fused_lora(gu.fused_lora, GATE_UP_NAMES, li, layers, s)
            if isinstance(o_proj, SyncRemoteLoRALinear):
                self._update_single_lora(o_proj, O_NAME, li, layers, s)
            if isinstance(down, SyncRemoteLoRALinear):
                self._update_single_lora(down, DOWN_NAME, li, layers, s)

    def _update_fused_lora(self, fused: FusedLoRA, names: Sequence[str], li: int, layers: dict, scaling: float):
        """Rewrite fused_A = cat(A_i^T * s) and the diagonal blocks of fused_B
        in place; a projection the new adapter lacks becomes a zero block."""
        if not fused.has_lora:
            return
        mods = [layers.get(li, {}).get(n) for n in names]
        if not any(m is not None for m in mods):
            return
        r = fused.rank
        fA, fB = fused.fused_A.data, fused.fused_B.data
        fB.zero_()
        col = 0
        for i, (m, d) in enumerate(zip(mods, fused.out_dims)):
            if m is None:
                fA[:, i * r:(i + 1) * r].zero_()
            else:
                fA[:, i * r:(i + 1) * r].copy_(m.lora_A["default"].weight.t() * scaling)
                fB[i * r:(i + 1) * r, col:col + d].copy_(m.lora_B["default"].weight.t())
            col += d

    def _update_single_lora(self, mod: SyncRemoteLoRALinear, name: str, li: int, layers: dict, scaling: float):
        m = layers.get(li, {}).get(name)
        if m is None:
            return
        mod.lora_A.weight.data.copy_(m.lora_A["default"].weight)
        mod.lora_B.weight.data.copy_(m.lora_B["default"].weight)
        mod.scaling = scaling

    # ---------------------------------------------------------- rank change
    def _zero_lora_modules(self, model):
        """Zero the outgoing adapter's tensors before they are released."""
        for _, qkv, gu, _, o_proj, _, down in _layer_slots(model):
            for h in (qkv, gu):
                fl = getattr(h, "fused_lora", None) if h is not None else None
                if fl is not None and fl.has_lora:
                    fl.fused_A.data.zero_()
                    fl.fused_B.data.zero_()
            for m in (o_proj, down):
                if isinstance(m, SyncRemoteLoRALinear):
                    m.lora_A.weight.data.zero_()
                    m.lora_B.weight.data.zero_()

    def _recreate_lora_modules(self, model, layers: dict, config: dict):
        self._zero_lora_modules(model)
        s = _scaling(config)
        hidden = self.info["hidden_size"]
        kv = hidden // self.info["num_heads"] * self.info["num_kv_heads"]
        qkv_dims = [hidden, kv, kv]
        gu_dims = [self.info["intermediate_size"]] * 2
        for li, qkv, gu, o_owner, o_proj, d_owner, down in _layer_slots(model):
            got = layers.get(li, {})
            if qkv is not None:
                mods = [got.get(n) for n in QKV_NAMES]
                qkv.fused_lora = FusedLoRA(mods, qkv_dims, self.device, self.dtype) if any(mods) else None
            if gu is not None:
                mods = [got.get(n) for n in GATE_UP_NAMES]
                gu.fused_lora = FusedLoRA(mods, gu_dims, self.device, self.dtype) if any(mods) else None
            for mod, name in ((o_proj, O_NAME), (down, DOWN_NAME)):
                if isinstance(mod, SyncRemoteLoRALinear) and got.get(name) is not None:
                    new = got[name]
                    mod.lora_A = new.lora_A["default"]
                    mod.lora_B = new.lora_B["default"]
                    mod.scaling = s


class AdapterPool:
    """Adapters resident in HBM for the aggregator's pooled rounds.

    dims: {'hidden': H, 'kv': kv_heads * head_dim, 'inter': I}.  An adapter
    occupies one pool entry per (layer, fused projection): lora_A of the
    projection's blocks stacked [nblk * r, in] and lora_B per block
    [cols, r] (what ext_aggregator.register_adapter takes), scale
    lora_alpha / r.  A projection the adapter does not target is a zero block.
    """

    def __init__(self, num_layers: int, dims: dict, device, dtype: torch.dtype = torch.bfloat16):
        from .. import ext_aggregator as agg
        self.agg = agg
        self.num_layers = num_layers
        self.dims = dict(dims)
        self.device = torch.device(device)
        self.dtype = dtype
        self.entries: Dict[int, Dict[Tuple[int, int], Tuple[torch.Tensor, List[torch.Tensor]]]] = {}
        self.meta: Dict[int, dict] = {}
        self._lock = threading.Lock()

    def _groups(self):
        H, KV, I = self.dims["hidden"], self.dims["kv"], self.dims["inter"]
        agg = self.agg
        return ((agg.OP_QKV_FUSED, QKV_NAMES, H, (H, KV, KV)), (agg.OP_O_PROJ, (O_NAME,), H, (H,)),
                (agg.OP_GATE_UP_FUSED, GATE_UP_NAMES, H, (I, I)), (agg.OP_DOWN_PROJ, (DOWN_NAME,), I, (H,)))

    def _tensors(self, layers: dict, rank: int):
        """{(layer, op): (A stacked, [B...])} on the pool's device."""
        out = {}
        for li in range(self.num_layers):
            got = layers.get(li, {})
            for op, names, k_in, cols in self._groups():
                a_rows, bs = [], []
                for n, c in zip(names, cols):
                    m = got.get(n)
                    if m is None:
                        a_rows.append(torch.zeros(rank, k_in, device=self.device, dtype=self.dtype))
                        bs.append(torch.zeros(c, rank, device=self.device, dtype=self.dtype))
                    else:
                        A, B = m.lora_A["default"].weight.data, m.lora_B["default"].weight.data
                        if tuple(A.shape) != (rank, k_in) or tuple(B.shape) != (c, rank):
                            raise ValueError(f"adapter layer {li} {n}: lora_A {tuple(A.shape)} / lora_B "
                                             f"{tuple(B.shape)} do not fit [{rank}, {k_in}] / [{c}, {rank}]")
                        a_rows.append(A.to(self.device, self.dtype))
                        bs.append(B.to(self.device, self.dtype).contiguous())
                out[(li, op)] = (torch.cat(a_rows, 0).contiguous(), bs)
        return out

    def load(self, adapter_id: int, lora_path: str) -> dict:
        """Load a PEFT adapter directory into the pool as `adapter_id`
        (replacing any adapter of that id)."""
        layers, config = load_lora_fast(lora_path, self.device, self.dtype)
        with self._lock:
            return self._install(adapter_id, layers, config, lora_path, in_place=False)

    def swap(self, adapter_id: int, lora_path: str) -> dict:
        """Hot swap adapter `adapter_id` to the one at `lora_path`.  Same
        rank: weights written into the resident tensors on the current stream
        (ordered after the rounds already queued there), pool pointers kept.
        Different rank: new tensors registered (recapture graphs)."""
        t0 = time.perf_counter()
        layers, config = load_lora_fast(lora_path, self.device, self.dtype)
        t1 = time.perf_counter()
        with self._lock:
            old = self.meta.get(adapter_id)
            in_place = old is not None and old["rank"] == config["r"]
            res = self._install(adapter_id, layers, config, lora_path, in_place=in_place)
        res.update({"old_adapter": old["path"] if old else None, "old_rank": old["rank"] if old else 0,
                    "load_time_ms": round((t1 - t0) * 1000, 2),
                    "total_time_ms": round((time.perf_counter() - t0) * 1000, 2)})
        return res

    def _install(self, adapter_id, layers, config, path, in_place):
        rank, scale = config["r"], _scaling(config)
        new = self._tensors(layers, rank)
        if in_place:
            cur = self.entries[adapter_id]
            for key, (A, Bs) in new.items():
                cA, cBs = cur[key]
                cA.copy_(A)
                for cb, b in zip(cBs, Bs):
                    cb.copy_(b)
            tensors = cur
        else:
            tensors = new
        for (li, op), (A, Bs) in tensors.items():
            self.agg.register_adapter(adapter_id, li, op, A, Bs, scale)
        self.entries[adapter_id] = tensors
        self.meta[adapter_id] = {"rank": rank, "scale": scale, "path": path}
        return {"success": True, "adapter_id": adapter_id, "new_adapter": path, "new_rank": rank,
                "in_place": in_place, "entries": len(tensors)}

    def adapters(self) -> Dict[int, dict]:
        with self._lock:
            return {k: dict(v) for k, v in self.meta.items()}
