"""Write synthetic LoRA adapters in PEFT's on-disk format.

Same command line and output as the reference's generate_adapters.py:1-208
(`--rank R | --mixed`, `--num`, `--out`, `--start`, `--base-model`,
`--symlink`): one directory lora-<i> per adapter holding
adapter_model.safetensors (fp32 lora_A [r, in] / lora_B [out, r] under
PEFT's base_model.model.model.layers.<l>.<module>.lora_{A,B}.weight keys)
and adapter_config.json (lora_alpha = r, so scaling 1.0).  lora_A is
Kaiming-uniform (bound 1 / sqrt(in)), lora_B N(0, 0.004^2), so the deltas
have the size of a lightly trained adapter.  --mixed cycles ranks through
the serving mix 8, 16, 8, 4, 8, 32, 8, 64, 8, 16.  Random streams are seeded
per rank (not bit-identical to the reference's; the format is).

    python -m swarmlora_amd.worker.generate_adapters --mixed --num 500 --out /data/adapters --symlink
"""

import argparse
import collections
import json
import math
import os
import shutil

import torch

# (in_features, out_features) per target module, per base model
_LLAMA8B = {
    "self_attn.q_proj": (4096, 4096),
    "self_attn.k_proj": (4096, 1024),
    "self_attn.v_proj": (4096, 1024),
    "self_attn.o_proj": (4096, 4096),
    "mlp.gate_proj": (4096, 14336),
    "mlp.up_proj": (4096, 14336),
    "mlp.down_proj": (14336, 4096),
}
MODEL_PRESETS = {
    "llama-3.1-8b": {"num_layers": 32, "modules": dict(_LLAMA8B)},
    "mistral-7b": {"num_layers": 32, "modules": dict(_LLAMA8B)},
    "llama-2-13b": {"num_layers": 40, "modules": {
        "self_attn.q_proj": (5120, 5120),
        "self_attn.k_proj": (5120, 5120),
        "self_attn.v_proj": (5120, 5120),
        "self_attn.o_proj": (5120, 5120),
        "mlp.gate_proj": (5120, 13824),
        "mlp.up_proj": (5120, 13824),
        "mlp.down_proj": (13824, 5120),
    }},
}
NUM_LAYERS = MODEL_PRESETS["llama-3.1-8b"]["num_layers"]
MODULES = MODEL_PRESETS["llama-3.1-8b"]["modules"]
MIXED_PATTERN = [8, 16, 8, 4, 8, 32, 8, 64, 8, 16]


def get_model_dims(base_model: str) -> dict:
    """Preset for a base-model name (13b -> Llama-2-13B, mistral -> Mistral-7B,
    anything else Llama-3.1-8B)."""
    name = base_model.lower()
    if "13b" in name:
        return MODEL_PRESETS["llama-2-13b"]
    if "mistral" in name:
        return MODEL_PRESETS["mistral-7b"]
    return MODEL_PRESETS["llama-3.1-8b"]


def get_mixed_rank(adapter_idx: int) -> int:
    return MIXED_PATTERN[adapter_idx % len(MIXED_PATTERN)]


def generate_adapter(rank: int, seed: int = 42, num_layers: int = NUM_LAYERS, modules: dict = None) -> dict:
    """{PEFT key: fp32 tensor} for one adapter of `rank`."""
    modules = MODULES if modules is None else modules
    g = torch.Generator().manual_seed(seed * 1000003 + rank)
    out = {}
    for layer in range(num_layers):
        for name, (fin, fout) in modules.items():
            key = f"base_model.model.model.layers.{layer}.{name}"
            bound = 1.0 / math.sqrt(fin)
            out[f"{key}.lora_A.weight"] = (torch.rand(rank, fin, generator=g) * 2 - 1) * bound
            out[f"{key}.lora_B.weight"] = torch.randn(fout, rank, generator=g) * 0.004
    return out


def make_config(rank: int, base_model: str = "meta-llama/Meta-Llama-3.1-8B-Instruct") -> dict:
    """adapter_config.json of a LoRA on all seven projections, lora_alpha = r."""
    return {
        "alpha_pattern": {},
        "auto_mapping": None,
        "base_model_name_or_path": base_model,
        "bias": "none",
        "fan_in_fan_out": False,
        "inference_mode": True,
        "init_lora_weights": True,
        "layer_replication": None,
        "layers_pattern": None,
        "layers_to_transform": None,
        "loftq_config": {},
        "lora_alpha": rank,
        "lora_dropout": 0,
        "megatron_config": None,
        "megatron_core": "megatron.core",
        "modules_to_save": None,
        "peft_type": "LORA",
        "r": rank,
        "rank_pattern": {},
        "revision": None,
        "target_modules": ["gate_proj", "down_proj", "up_proj", "o_proj", "q_proj", "k_proj", "v_proj"],
        "task_type": "CAUSAL_LM",
        "use_dora": False,
        "use_rslora": False,
    }


def write_adapter(path: str, weights: dict, config: dict):
    from safetensors.torch import save_file
    os.makedirs(path, exist_ok=True)
    save_file({k: v.contiguous() for k, v in weights.items()}, os.path.join(path, "adapter_model.safetensors"))
    with open(os.path.join(path, "adapter_config.json"), "w") as f:
        json.dump(config, f, indent=2)


def generate(out: str, num: int, rank=None, mixed: bool = False, start: int = 0,
             base_model: str = "meta-llama/Meta-Llama-3.1-8B-Instruct", symlink: bool = False,
             num_layers=None, modules=None, seed: int = 42) -> dict:
    """Write adapters lora-<start> .. lora-<start+num-1> under `out`.  One set
    of weights per rank (adapters of the same rank share it, as in the
    reference); with symlink only the first adapter of each rank is written
    and the others link to it.  Returns {rank: count}."""
    if not mixed and rank is None:
        raise ValueError("either rank or mixed is required")
    dims = get_model_dims(base_model)
    num_layers = dims["num_layers"] if num_layers is None else num_layers
    modules = dims["modules"] if modules is None else modules
    ranks = sorted(set(MIXED_PATTERN)) if mixed else [rank]
    cache = {r: generate_adapter(r, seed, num_layers, modules) for r in ranks}
    counts, first = collections.Counter(), {}
    for i in range(num):
        idx = start + i
        r = get_mixed_rank(idx) if mixed else rank
        counts[r] += 1
        d = os.path.join(out, f"lora-{idx}")
        if symlink and r in first:
            if os.path.islink(d):
                os.unlink(d)
            elif os.path.exists(d):
                shutil.rmtree(d)
            os.symlink(os.path.relpath(first[r], os.path.dirname(d)), d)
            continue
        write_adapter(d, cache[r], make_config(r, base_model))
        first[r] = d
    return dict(counts)


def main(argv=None):
    ap = argparse.ArgumentParser(description="Generate synthetic LoRA adapters (PEFT safetensors)")
    ap.add_argument("--rank", type=int, default=None, help="LoRA rank of a uniform pool")
    ap.add_argument("--mixed", action="store_true", help="round-robin mixed ranks")
    ap.add_argument("--num", type=int, default=50, help="number of adapters")
    ap.add_argument("--out", type=str, required=True, help="output directory")
    ap.add_argument("--start", type=int, default=0, help="first lora-N index")
    ap.add_argument("--base-model", type=str, default="meta-llama/Meta-Llama-3.1-8B-Instruct")
    ap.add_argument("--symlink", action="store_true", help="write one adapter per rank, link the rest")
    args = ap.parse_args(argv)
    if not args.mixed and args.rank is None:
        ap.error("Either --rank or --mixed is required")
    counts = generate(args.out, args.num, args.rank, args.mixed, args.start, args.base_model, args.symlink)
    dist = ", ".join(f"r{r}:{c}" for r, c in sorted(counts.items()))
    print(f"Generated {args.num} adapters in {args.out} ({dist})")


if __name__ == "__main__":
    main()
