"""Worker-side LoRA modules on the libswl kernels.

Same classes, constructor arguments and attributes as the reference's
src/worker/model_builder.py (FastLoRAModule :27-45, SyncRemoteLinear :186-190,
SyncRemoteLoRALinear :193-201, FusedLoRA :217-262, SyncFusedQKV/GateUp
:265-277) plus the PEFT safetensors loader (load_lora_fast :141-183, local
directories only: there is no hub access).  Every product runs through
libswl (bf16 operands, fp32 accumulation, bf16 results), never torch matmul.
"""

import json
import os
from typing import Dict, Optional, Sequence

import torch
import torch.nn as nn

from .. import ops

OP_O_PROJ = 3
OP_DOWN_PROJ = 6
OP_QKV_FUSED = 9
OP_GATE_UP_FUSED = 10
OP_EMBED = 11
OP_LM_HEAD = 12


def _as2d(x: torch.Tensor) -> torch.Tensor:
    x2 = x.reshape(-1, x.shape[-1])
    return x2 if x2.stride(-1) == 1 else x2.contiguous()


class HipLinear(nn.Module):
    """Bias-free linear layer y = x @ weight.T computed by libswl (the
    nn.Linear the reference builds for lora_A / lora_B)."""

    def __init__(self, weight: torch.Tensor):
        super().__init__()
        self.weight = nn.Parameter(weight, requires_grad=False)

    @property
    def in_features(self):
        return self.weight.shape[1]

    @property
    def out_features(self):
        return self.weight.shape[0]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x2 = _as2d(x)
        w = self.weight.data
        if x2.is_contiguous() and w.is_contiguous() and w.shape[1] % 32 == 0 and x2.shape[0] > 0:
            y = ops.gemm(x2, w)
        else:
            y = ops.matmul(x2, w, trans_b=True)
        return y.reshape(*x.shape[:-1], w.shape[0])


class FastLoRAModule:
    """Mimics PEFT's LoraLayer bookkeeping for one projection
    (model_builder.py:27-45): lora_A [r, in], lora_B [out, r], scaling."""

    def __init__(self, lora_A: torch.Tensor, lora_B: torch.Tensor, scaling: float):
        self.lora_A = {"default": HipLinear(lora_A)}
        self.lora_B = {"default": HipLinear(lora_B)}
        self.scaling = {"default": scaling}
        self.lora_dropout = {"default": nn.Identity()}


def _rows_fit(x2: torch.Tensor, nr: int) -> bool:
    """A worker's LoRA delta fits one lora_rows launch: at most 4 token rows
    of 16-byte multiples, 16-byte aligned, at most 64 shrink columns."""
    return (0 < x2.shape[0] <= ops.LORA_ROWS_MAX and nr <= ops.LORA_ROWS_MAX_NR and x2.stride(1) == 1 and
            x2.shape[1] % 8 == 0 and x2.stride(0) % 8 == 0 and x2.data_ptr() % 16 == 0)


class SyncRemoteLinear(nn.Module):
    """Placeholder for a projection the aggregator computes (no adapter)."""

    def __init__(self, op: int, layer: int, out_dim: int):
        super().__init__()
        self.op, self.layer, self.out_dim = op, layer, out_dim


class SyncRemoteLoRALinear(nn.Module):
    """Aggregator-computed O / Down projection with a worker-side adapter."""

    def __init__(self, op: int, layer: int, out_dim: int, lora_module):
        super().__init__()
        self.op, self.layer, self.out_dim = op, layer, out_dim
        self.lora_A = lora_module.lora_A["default"]
        self.lora_B = lora_module.lora_B["default"]
        self.scaling = lora_module.scaling["default"]
        self.dropout = lora_module.lora_dropout["default"]

    def delta(self, x: torch.Tensor) -> torch.Tensor:
        """lora_B(lora_A(dropout(x))) * scaling (worker_sync.py:305, :375),
        with the scaling applied before the single bf16 rounding; a decode
        token's few rows take one lora_rows launch."""
        x2 = _as2d(self.dropout(x))
        A, B = self.lora_A.weight.data, self.lora_B.weight.data
        if _rows_fit(x2, A.shape[0]):
            y = ops.lora_rows(x2, A, False, [(B, B.shape[0], False)], A.shape[0], float(self.scaling))
        else:
            u = self.lora_A(x2)
            y = ops.matmul(u, B, trans_b=True, alpha=float(self.scaling))
        return y.reshape(*x.shape[:-1], y.shape[-1])


class FusedLoRA(nn.Module):
    """Fused LoRA of several projections sharing one input (QKV or Gate+Up):
    fused_A = cat_i(A_i^T * s_i) [in, n*r] and a block-diagonal fused_B
    [n*r, sum(out_dims)] (model_builder.py:217-256).  forward returns the
    per-projection deltas (x @ fused_A) @ fused_B split by out_dims; only the
    diagonal blocks of fused_B are read."""

    def __init__(self, lora_modules: list, out_dims: list, device, dtype: torch.dtype):
        super().__init__()
        self.out_dims = list(out_dims)
        self.num_loras = len(lora_modules)
        valid = [m for m in lora_modules if m is not None]
        if not valid:
            self.has_lora = False
            return
        self.has_lora = True
        a_w, b_w = [], []
        first_A = valid[0].lora_A["default"].weight
        for i, m in enumerate(lora_modules):
            if m is not None and hasattr(m, "lora_A"):
                A = m.lora_A["default"].weight
                B = m.lora_B["default"].weight
                s = m.scaling["default"]
                a_w.append(A.t() * s)
                b_w.append(B.t())
            else:
                a_w.append(torch.zeros(first_A.size(1), first_A.size(0), device=device, dtype=dtype))
                b_w.append(torch.zeros(first_A.size(0), self.out_dims[i], device=device, dtype=dtype))
        self.fused_A = nn.Parameter(torch.cat(a_w, dim=1).contiguous(), requires_grad=False)
        self.rank = a_w[0].size(1)
        fused_B = torch.zeros(self.rank * self.num_loras, sum(self.out_dims), device=device, dtype=dtype)
        col = 0
        for i, B in enumerate(b_w):
            fused_B[i * self.rank:(i + 1) * self.rank, col:col + self.out_dims[i]] = B
            col += self.out_dims[i]
        self.fused_B = nn.Parameter(fused_B, requires_grad=False)
        self.dropout = valid[0].lora_dropout["default"]

    def forward(self, x: torch.Tensor) -> list:
        if not self.has_lora:
            return [None] * self.num_loras
        x2 = _as2d(self.dropout(x))
        fA, fB, r = self.fused_A.data, self.fused_B.data, self.rank
        if _rows_fit(x2, fA.shape[1]) and len(self.out_dims) <= 4:
            # a decode token's rows: shrink and every block's expand in one launch
            blocks, col = [], 0
            for i, d in enumerate(self.out_dims):
                blocks.append((fB[i * r:(i + 1) * r, col:col + d], d, True))
                col += d
            delta = ops.lora_rows(x2, fA, True, blocks, r)
        else:
            u = ops.matmul(x2, fA, trans_b=False)            # [m, n*r] bf16
            delta = torch.empty(x2.shape[0], sum(self.out_dims), dtype=x2.dtype, device=x2.device)
            col = 0
            for i, d in enumerate(self.out_dims):
                ops.matmul(u[:, i * r:(i + 1) * r], fB[i * r:(i + 1) * r, col:col + d], trans_b=False,
                           out=delta[:, col:col + d])
                col += d
        delta = delta.reshape(*x.shape[:-1], delta.shape[-1])
        return list(delta.split(self.out_dims, dim=-1))


class SyncFusedQKV(nn.Module):
    def __init__(self, layer: int, dims: list, fused_lora: Optional[FusedLoRA] = None):
        super().__init__()
        self.layer, self.dims, self.fused_lora = layer, dims, fused_lora


class SyncFusedGateUp(nn.Module):
    def __init__(self, layer: int, dims: list, fused_lora: Optional[FusedLoRA] = None):
        super().__init__()
        self.layer, self.dims, self.fused_lora = layer, dims, fused_lora


def load_lora_fast(lora_path: str, device, dtype: torch.dtype):
    """PEFT adapter directory -> ({layer: {module: FastLoRAModule}}, config)
    (model_builder.py:141-183).  Keys look like
    base_model.model.model.layers.{i}.{self_attn|mlp}.{proj}.lora_{A|B}.weight;
    scaling = lora_alpha / r.  Only safetensors is accepted."""
    from safetensors import safe_open
    if not os.path.isdir(lora_path):
        raise FileNotFoundError(f"adapter directory not found: {lora_path}")
    with open(os.path.join(lora_path, "adapter_config.json")) as f:
        config = json.load(f)
    st_file = os.path.join(lora_path, "adapter_model.safetensors")
    if not os.path.exists(st_file):
        if os.path.exists(os.path.join(lora_path, "adapter_model.bin")):
            raise ValueError(f"Adapter at {lora_path!r} uses .bin format which is not allowed. "
                             "Convert to safetensors format.")
        raise FileNotFoundError(f"No adapter weights found in {lora_path}")
    weights = {}
    with safe_open(st_file, framework="pt", device="cpu") as f:
        for key in f.keys():
            weights[key] = f.get_tensor(key).to(dtype=dtype).to(device)
    rank = config["r"]
    scaling = config.get("lora_alpha", rank) / rank
    raw: Dict[int, Dict[str, dict]] = {}
    for key, t in weights.items():
        parts = key.split(".")
        layer = int(parts[4])
        module = parts[5] + "." + parts[6]
        kind = parts[-2]
        raw.setdefault(layer, {}).setdefault(module, {})[kind] = t
    out = {layer: {m: FastLoRAModule(ab["lora_A"], ab["lora_B"], scaling) for m, ab in mods.items()}
           for layer, mods in raw.items()}
    return out, config


def pool_tensors(modules: Sequence[Optional[FastLoRAModule]]):
    """Stacked lora_A [n*r, in] (scaling folded into the pool's scale, not
    into A) and the per-block lora_B list of a fused projection, for
    ext_aggregator.register_adapter.  Returns (a, [b...], rank, scale)."""
    valid = [m for m in modules if m is not None]
    if not valid:
        return None
    A0 = valid[0].lora_A["default"].weight
    rank, in_dim = A0.shape
    scale = valid[0].scaling["default"]
    a_rows, bs = [], []
    for m in modules:
        if m is None:
            raise ValueError("pooled fused adapters need every projection (a missing one is a zero block)")
        if abs(m.scaling["default"] - scale) > 0:
            raise ValueError("pooled fused adapters share one scaling")
        a_rows.append(m.lora_A["default"].weight.data)
        bs.append(m.lora_B["default"].weight.data.contiguous())
    return torch.cat(a_rows, 0).contiguous(), bs, rank, scale
