"""A small Llama-shaped model (head_dim 128, GQA) built from fixed seeds, plus
its CPU-oracle forward, for the end-to-end multi-process test."""

from types import SimpleNamespace

import torch

from tests._util import BF16, randn

CFG = SimpleNamespace(hidden=512, heads=4, kv_heads=2, head_dim=128, inter=1024, vocab=640, layers=2, eps=1e-5,
                      theta=500000.0, rank=8, scale=2.0, block=16, max_seq=256, chunk=16)
QKV = CFG.hidden + 2 * CFG.kv_heads * CFG.head_dim
KVD = CFG.kv_heads * CFG.head_dim
PROJ = {  # name: (in, out)
    "self_attn.q_proj": (CFG.hidden, CFG.hidden), "self_attn.k_proj": (CFG.hidden, KVD),
    "self_attn.v_proj": (CFG.hidden, KVD), "self_attn.o_proj": (CFG.hidden, CFG.hidden),
    "mlp.gate_proj": (CFG.hidden, CFG.inter), "mlp.up_proj": (CFG.hidden, CFG.inter),
    "mlp.down_proj": (CFG.inter, CFG.hidden),
}


def base_weights():
    """CPU bf16 weights: per layer dict of q,k,v,o,gate,up,down and the two
    norm vectors; embed, lm_head and the final norm."""
    layers = []
    for li in range(CFG.layers):
        s = 1000 * (li + 1)
        w = {name.split(".")[1][:-5]: randn((o, i), s + j, std=0.02) for j, (name, (i, o)) in enumerate(PROJ.items())}
        w["input_norm"] = (1 + randn((CFG.hidden,), s + 50, std=0.1).float()).to(BF16)
        w["post_norm"] = (1 + randn((CFG.hidden,), s + 51, std=0.1).float()).to(BF16)
        layers.append(w)
    return {"layers": layers, "embed": randn((CFG.vocab, CFG.hidden), 7, std=1.0),
            "lm_head": randn((CFG.vocab, CFG.hidden), 8, std=0.02),
            "final_norm": (1 + randn((CFG.hidden,), 9, std=0.1).float()).to(BF16)}


def adapter(worker_id):
    """{layer: {proj_name: (A [r, in], B [out, r])}} for one worker."""
    out = {}
    for li in range(CFG.layers):
        out[li] = {}
        for j, (name, (i, o)) in enumerate(PROJ.items()):
            s = 100000 * (worker_id + 1) + 100 * li + 2 * j
            out[li][name] = (randn((CFG.rank, i), s, std=0.02), randn((o, CFG.rank), s + 1, std=0.02))
    return out


def oracle_steps(weights, ad, steps):
    """Teacher-forced CPU oracle: steps is the list of [1, t] input id
    tensors the worker fed; returns the final-norm hidden of each step."""
    from oracle import reference_path as ref
    c = CFG
    inv = ref.rope_inv_freq(c.head_dim, c.theta)
    cs = ref.cos_sin_cache(inv, c.max_seq)
    nblk = c.max_seq // c.block
    kc = [torch.zeros(nblk, c.block, c.kv_heads, c.head_dim, dtype=BF16) for _ in range(c.layers)]
    vc = [torch.zeros(nblk, c.block, c.kv_heads, c.head_dim, dtype=BF16) for _ in range(c.layers)]
    bt = torch.arange(nblk, dtype=torch.int32).reshape(1, nblk)
    seqlen = 0
    outs = []
    dims_qkv = [c.hidden, KVD, KVD]
    for ids in steps:
        t = ids.shape[1]
        h = weights["embed"][ids.reshape(-1).clamp(0, c.vocab - 1)].reshape(1, t, c.hidden)
        for li, w in enumerate(weights["layers"]):
            a = ad[li]
            res = h
            hn = ref.rms_norm(h, w["input_norm"], c.eps)
            Wqkv, Wgu = ref.fuse_layer_weights(w["q"], w["k"], w["v"], w["gate"], w["up"])
            base = ref.base_gemm(hn.reshape(t, -1), Wqkv)
            fA, fB = ref.fused_lora_weights([(*a[n], c.scale) for n in ("self_attn.q_proj", "self_attn.k_proj",
                                                                         "self_attn.v_proj")], dims_qkv)
            q, k, v = ref.qkv_get(base, dims_qkv, ref.fused_lora_forward(hn.reshape(t, -1), fA, fB, dims_qkv))
            sl = torch.tensor([seqlen], dtype=torch.int32)
            pos = torch.arange(seqlen, seqlen + t)
            attn, _, _ = ref.paged_attention(q.reshape(1, t, c.heads, c.head_dim),
                                             k.reshape(1, t, c.kv_heads, c.head_dim),
                                             v.reshape(1, t, c.kv_heads, c.head_dim), kc[li], vc[li], bt, sl, pos, cs,
                                             1.0 / c.head_dim ** 0.5)
            x = attn.reshape(t, -1)
            o = ref.base_gemm(x, w["o"])
            h = ref.o_down_get(o, res.reshape(t, -1), ref.remote_lora_delta(x, *a["self_attn.o_proj"], c.scale))
            h = h.reshape(1, t, -1)
            res = h
            hn = ref.rms_norm(h, w["post_norm"], c.eps).reshape(t, -1)
            gu = ref.base_gemm(hn, Wgu)
            fA, fB = ref.fused_lora_weights([(*a[n], c.scale) for n in ("mlp.gate_proj", "mlp.up_proj")],
                                            [c.inter, c.inter])
            g, u = ref.qkv_get(gu, [c.inter, c.inter], ref.fused_lora_forward(hn, fA, fB, [c.inter, c.inter]))
            m = ref.silu_mul(g, u)
            d = ref.base_gemm(m, w["down"])
            h = ref.o_down_get(d, res.reshape(t, -1), ref.remote_lora_delta(m, *a["mlp.down_proj"], c.scale))
            h = h.reshape(1, t, -1)
        seqlen += t
        outs.append(ref.rms_norm(h, weights["final_norm"], c.eps))
    return outs
