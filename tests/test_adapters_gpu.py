"""GPU test of the HBM adapter pool: adapters loaded from PEFT directories
into the aggregator's pool drive the pooled rounds; an equal-rank hot swap
rewrites the resident tensors in place (pool pointers unchanged) and a rank
change re-registers; each round checked against the oracle with the adapter
then in the pool."""

import os

import pytest
import torch

from oracle import reference_path as ref
from tests._util import BF16, assert_close, randn

pytestmark = pytest.mark.gpu

H, I, KV, D = 1024, 2048, 2, 128
MODS = {"self_attn.q_proj": (H, H), "self_attn.k_proj": (H, KV * D), "self_attn.v_proj": (H, KV * D),
        "self_attn.o_proj": (H, H), "mlp.gate_proj": (H, I), "mlp.up_proj": (H, I), "mlp.down_proj": (I, H)}


def test_pool_load_swap_in_place_and_rank_change(dev, tmp_path):
    from swarmlora_amd import ext_aggregator as agg
    from swarmlora_amd.worker import generate_adapters as gen
    from swarmlora_amd.worker.adapter_manager import AdapterPool

    paths = {}
    for name, r, seed in (("a", 8, 1), ("b", 8, 2), ("c", 16, 3)):
        w = gen.generate_adapter(r, seed=seed, num_layers=1, modules=MODS)
        cfg = gen.make_config(r)
        cfg["lora_alpha"] = 2 * r   # scaling 2.0
        paths[name] = (os.path.join(str(tmp_path), name), w, r)
        gen.write_adapter(paths[name][0], w, cfg)

    agg.init_slot_pool(2, 0, H, I, KV, D, 4, 2)
    try:
        wts = {n: randn(s, 40 + i, std=0.02) for i, (n, s) in enumerate(
            [("q", (H, H)), ("k", (KV * D, H)), ("v", (KV * D, H)), ("o", (H, H)), ("gate", (I, H)), ("up", (I, H)),
             ("down", (H, I))])}
        agg.init_aggregator_begin(1, 0)
        agg.init_aggregator_layer(0, *(wts[n].to(dev) for n in ("q", "k", "v", "o")), torch.empty(0),
                                  wts["gate"].to(dev), wts["up"].to(dev), wts["down"].to(dev), torch.empty(0))
        agg.init_aggregator_finalize()
        for wid in range(2):
            agg.claim_slot(wid)
        pool = AdapterPool(1, {"hidden": H, "kv": KV * D, "inter": I}, dev)

        def check(name):
            _, w, r = paths[name]
            key = "base_model.model.model.layers.0.{}.lora_{}.weight"
            for op, names, k_in, dims, W in (
                    (agg.OP_QKV_FUSED, ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"), H,
                     [H, KV * D, KV * D], torch.cat([wts["q"], wts["k"], wts["v"]], 0)),
                    (agg.OP_DOWN_PROJ, ("mlp.down_proj",), I, [H], wts["down"])):
                x = randn((3, k_in), 77 + op)
                sin, _ = agg.slot_tensors(0)
                sin[: 3 * k_in].copy_(x.reshape(-1).to(dev))
                agg.execute_round(op, 0, [0], [0], [3], [5])
                torch.cuda.synchronize()
                ad = [[(w[key.format(n, "A")].to(BF16), w[key.format(n, "B")].to(BF16), 2.0) for n in names]]
                want = ref.round_with_lora(op, [x], [3], W, ad, dims)[0]
                _, sout = agg.slot_tensors(0)
                assert_close(sout[: 3 * sum(dims)].reshape(3, sum(dims)), want, what=f"{name} op {op}")

        res = pool.load(5, paths["a"][0])
        assert res["success"] and res["new_rank"] == 8 and res["entries"] == 4
        check("a")
        ptrs = {k: (A.data_ptr(), [b.data_ptr() for b in Bs]) for k, (A, Bs) in pool.entries[5].items()}
        res = pool.swap(5, paths["b"][0])
        assert res["in_place"] and res["old_rank"] == 8
        assert {k: (A.data_ptr(), [b.data_ptr() for b in Bs]) for k, (A, Bs) in pool.entries[5].items()} == ptrs
        check("b")
        res = pool.swap(5, paths["c"][0])
        assert not res["in_place"] and res["new_rank"] == 16
        check("c")
        assert pool.adapters()[5]["rank"] == 16
    finally:
        agg.clear_adapters()
        for wid in range(2):
            agg.release_slot(wid, wid)
        agg.cleanup_slot_pool()
