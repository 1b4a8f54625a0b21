"""Adapter format, generation and hot swap on the CPU (no kernel calls).

The generator writes PEFT's layout (generate_adapters.py in the reference);
load_lora_fast reads it back; AdapterManager swaps a worker model's LoRA
modules in place at equal rank and rebuilds them when the rank changes
(adapter_manager.py:47-280), with the same result dictionary.
"""

import json
import os
from types import SimpleNamespace

import pytest
import torch

from swarmlora_amd.worker import generate_adapters as gen
from swarmlora_amd.worker.adapter_manager import AdapterManager
from swarmlora_amd.worker.model_builder import FusedLoRA, SyncRemoteLoRALinear, load_lora_fast

H, KV, I, L = 64, 32, 96, 2
MODS = {"self_attn.q_proj": (H, H), "self_attn.k_proj": (H, KV), "self_attn.v_proj": (H, KV),
        "self_attn.o_proj": (H, H), "mlp.gate_proj": (H, I), "mlp.up_proj": (H, I), "mlp.down_proj": (I, H)}
INFO = {"hidden_size": H, "num_heads": 4, "num_kv_heads": 2, "intermediate_size": I}


def _write(tmp, name, rank, seed, drop=()):
    w = gen.generate_adapter(rank, seed=seed, num_layers=L, modules=MODS)
    w = {k: v for k, v in w.items() if not any(d in k for d in drop)}
    path = os.path.join(tmp, name)
    gen.write_adapter(path, w, gen.make_config(rank))
    return path, w


def test_generated_adapter_round_trips_through_load_lora_fast(tmp_path):
    path, w = _write(str(tmp_path), "a", 8, 1)
    cfg = json.load(open(os.path.join(path, "adapter_config.json")))
    assert cfg["r"] == 8 and cfg["lora_alpha"] == 8 and cfg["peft_type"] == "LORA"
    assert len(w) == L * len(MODS) * 2
    layers, config = load_lora_fast(path, "cpu", torch.float32)
    assert sorted(layers) == list(range(L)) and config["r"] == 8
    for li in range(L):
        assert sorted(layers[li]) == sorted(MODS)
        for m, (fin, fout) in MODS.items():
            mod = layers[li][m]
            A = mod.lora_A["default"].weight
            B = mod.lora_B["default"].weight
            assert tuple(A.shape) == (8, fin) and tuple(B.shape) == (fout, 8)
            assert torch.equal(A, w[f"base_model.model.model.layers.{li}.{m}.lora_A.weight"])
            assert mod.scaling["default"] == 1.0
            assert float(A.abs().max()) <= 1.0 / fin ** 0.5 + 1e-7   # Kaiming-uniform bound


def test_generate_mixed_ranks_and_symlinks(tmp_path):
    out = str(tmp_path)
    counts = gen.generate(out, 12, mixed=True, symlink=True, num_layers=1, modules=MODS)
    assert counts == {8: 6, 16: 3, 4: 1, 32: 1, 64: 1}
    for i in range(12):
        d = os.path.join(out, f"lora-{i}")
        _, cfg = load_lora_fast(d, "cpu", torch.float32)
        assert cfg["r"] == gen.get_mixed_rank(i)
    assert os.path.islink(os.path.join(out, "lora-2")) and not os.path.islink(os.path.join(out, "lora-0"))
    assert gen.get_model_dims("meta-llama/Llama-2-13b-hf")["num_layers"] == 40
    with pytest.raises(ValueError):
        gen.generate(out, 1)


def _model(path):
    """A reference-shaped hollow model (model.model.layers[i].self_attn / .mlp)
    built from an adapter directory with this package's LoRA modules."""
    layers, _ = load_lora_fast(path, "cpu", torch.float32)
    out = []
    for li in range(L):
        g = layers[li]
        attn = SimpleNamespace(
            _fused_qkv=SimpleNamespace(fused_lora=FusedLoRA([g[n] for n in ("self_attn.q_proj", "self_attn.k_proj",
                                                                             "self_attn.v_proj")],
                                                            [H, KV, KV], "cpu", torch.float32)),
            o_proj=SyncRemoteLoRALinear(3, li, H, g["self_attn.o_proj"]))
        mlp = SimpleNamespace(
            _fused_gate_up=SimpleNamespace(fused_lora=FusedLoRA([g["mlp.gate_proj"], g["mlp.up_proj"]], [I, I], "cpu",
                                                                torch.float32)),
            down_proj=SyncRemoteLoRALinear(6, li, H, g["mlp.down_proj"]))
        out.append(SimpleNamespace(self_attn=attn, mlp=mlp))
    return SimpleNamespace(model=SimpleNamespace(layers=out))


def _fused_ref(w, li, names, dims, r, s):
    A = torch.cat([w[f"base_model.model.model.layers.{li}.{n}.lora_A.weight"].t() * s for n in names], 1)
    B = torch.zeros(r * len(names), sum(dims))
    col = 0
    for i, (n, d) in enumerate(zip(names, dims)):
        B[i * r:(i + 1) * r, col:col + d] = w[f"base_model.model.model.layers.{li}.{n}.lora_B.weight"].t()
        col += d
    return A, B


def test_swap_same_rank_in_place_then_rank_change(tmp_path):
    tmp = str(tmp_path)
    pa, _ = _write(tmp, "a", 8, 1)
    pb, wb = _write(tmp, "b", 8, 2, drop=("self_attn.k_proj",))
    pc, wc = _write(tmp, "c", 16, 3)
    model = _model(pa)
    mgr = AdapterManager(0, "cpu", torch.float32, INFO)
    mgr.set_adapter(pa, 8, {"r": 8})
    fl = model.model.layers[1].self_attn._fused_qkv.fused_lora
    ptr_a, ptr_o = fl.fused_A.data_ptr(), model.model.layers[1].self_attn.o_proj.lora_A.weight.data_ptr()

    res = mgr.swap_adapter(pb, model)
    assert res["success"] and not res["rank_changed"] and res["old_rank"] == 8 and res["new_rank"] == 8
    assert set(res) >= {"old_adapter", "new_adapter", "load_time_ms", "update_time_ms", "total_time_ms"}
    assert fl.fused_A.data_ptr() == ptr_a  # in place
    assert model.model.layers[1].self_attn.o_proj.lora_A.weight.data_ptr() == ptr_o
    # k_proj is missing from b: its blocks become zero
    wb_full = dict(wb)
    for li in range(L):
        for t in ("A", "B"):
            shape = (8, H) if t == "A" else (KV, 8)
            wb_full[f"base_model.model.model.layers.{li}.self_attn.k_proj.lora_{t}.weight"] = torch.zeros(shape)
    A, B = _fused_ref(wb_full, 1, ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"), [H, KV, KV], 8, 1.0)
    assert torch.equal(fl.fused_A.data, A) and torch.equal(fl.fused_B.data, B)
    assert torch.equal(model.model.layers[0].mlp.down_proj.lora_B.weight,
                       wb["base_model.model.model.layers.0.mlp.down_proj.lora_B.weight"])
    assert mgr.get_current_adapter() == pb and not mgr.is_swapping()

    res = mgr.swap_adapter(pc, model)
    assert res["success"] and res["rank_changed"] and res["new_rank"] == 16
    fl2 = model.model.layers[1].mlp._fused_gate_up.fused_lora
    A, B = _fused_ref(wc, 1, ("mlp.gate_proj", "mlp.up_proj"), [I, I], 16, 1.0)
    assert fl2.rank == 16 and torch.equal(fl2.fused_A.data, A) and torch.equal(fl2.fused_B.data, B)
    assert torch.equal(model.model.layers[1].self_attn.o_proj.lora_A.weight,
                       wc["base_model.model.model.layers.1.self_attn.o_proj.lora_A.weight"])


def test_swap_failure_reports_and_keeps_model(tmp_path):
    tmp = str(tmp_path)
    pa, _ = _write(tmp, "a", 8, 1)
    model = _model(pa)
    before = model.model.layers[0].self_attn._fused_qkv.fused_lora.fused_A.data.clone()
    mgr = AdapterManager(0, "cpu", torch.float32, INFO)
    mgr.set_adapter(pa, 8, {"r": 8})
    res = mgr.swap_adapter(os.path.join(tmp, "missing"), model)
    assert res["success"] is False and "not found" in res["error"]
    assert mgr.get_current_adapter() == pa
    assert torch.equal(model.model.layers[0].self_attn._fused_qkv.fused_lora.fused_A.data, before)
