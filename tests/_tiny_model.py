"""Llama-shaped test models built from fixed seeds, plus their CPU-oracle
forward, for the end-to-end multi-process tests: CFG is small (hidden 512,
GQA 4/2, two layers); WIDE has Llama-3.1-8B's widths (hidden 4096, 32 query /
8 kv heads of 128, intermediate 14336, rank-16 adapters) with two layers and
a 32000-entry vocabulary."""

from types import SimpleNamespace

import torch

from tests._util import BF16, randn

CFG = SimpleNamespace(hidden=512, heads=4, kv_heads=2, head_dim=128, inter=1024, vocab=640, layers=2, eps=1e-5,
                      theta=500000.0, rank=8, scale=2.0, block=16, max_seq=256, chunk=16)
WIDE = SimpleNamespace(hidden=4096, heads=32, kv_heads=8, head_dim=128, inter=14336, vocab=32000, layers=2, eps=1e-5,
                       theta=500000.0, rank=16, scale=2.0, block=16, max_seq=256, chunk=16)
CFGS = {"tiny": CFG, "wide": WIDE}
QKV = CFG.hidden + 2 * CFG.kv_heads * CFG.head_dim
KVD = CFG.kv_heads * CFG.head_dim


def proj_dims(c=CFG):
    """name: (in, out) of every projection of config c."""
    kvd = c.kv_heads * c.head_dim
    return {"self_attn.q_proj": (c.hidden, c.hidden), "self_attn.k_proj": (c.hidden, kvd),
            "self_attn.v_proj": (c.hidden, kvd), "self_attn.o_proj": (c.hidden, c.hidden),
            "mlp.gate_proj": (c.hidden, c.inter), "mlp.up_proj": (c.hidden, c.inter),
            "mlp.down_proj": (c.inter, c.hidden)}


PROJ = proj_dims(CFG)


def norm_weights(c=CFG):
    """The RMSNorm vectors of base_weights(c) alone: [(input, post) per
    layer], final (the same seeds, without drawing the projections)."""
    layers = [((1 + randn((c.hidden,), 1000 * (li + 1) + 50, std=0.1).float()).to(BF16),
               (1 + randn((c.hidden,), 1000 * (li + 1) + 51, std=0.1).float()).to(BF16)) for li in range(c.layers)]
    return layers, (1 + randn((c.hidden,), 9, std=0.1).float()).to(BF16)


def base_weights(c=CFG):
    """CPU bf16 weights: per layer dict of q,k,v,o,gate,up,down and the two
    norm vectors; embed, lm_head and the final norm."""
    layers = []
    for li in range(c.layers):
        s = 1000 * (li + 1)
        w = {name.split(".")[1][:-5]: randn((o, i), s + j, std=0.02)
             for j, (name, (i, o)) in enumerate(proj_dims(c).items())}
        w["input_norm"] = (1 + randn((c.hidden,), s + 50, std=0.1).float()).to(BF16)
        w["post_norm"] = (1 + randn((c.hidden,), s + 51, std=0.1).float()).to(BF16)
        layers.append(w)
    return {"layers": layers, "embed": randn((c.vocab, c.hidden), 7, std=1.0),
            "lm_head": randn((c.vocab, c.hidden), 8, std=0.02),
            "final_norm": (1 + randn((c.hidden,), 9, std=0.1).float()).to(BF16)}


def adapter(worker_id, c=CFG):
    """{layer: {proj_name: (A [r, in], B [out, r])}} for one worker."""
    out = {}
    for li in range(c.layers):
        out[li] = {}
        for j, (name, (i, o)) in enumerate(proj_dims(c).items()):
            s = 100000 * (worker_id + 1) + 100 * li + 2 * j
            out[li][name] = (randn((c.rank, i), s, std=0.02), randn((o, c.rank), s + 1, std=0.02))
    return out


def to_float32(weights, ad):
    """The same weights and adapter in float32 (exact conversions)."""
    w32 = {"layers": [{k: v.float() for k, v in lw.items()} for lw in weights["layers"]],
           "embed": weights["embed"].float(), "lm_head": weights["lm_head"].float(),
           "final_norm": weights["final_norm"].float()}
    return w32, {li: {n: (a.float(), b.float()) for n, (a, b) in m.items()} for li, m in ad.items()}


def oracle_steps(weights, ad, steps, c=CFG):
    """Teacher-forced CPU oracle: steps is the list of [1, t] input id
    tensors the worker fed; returns the final-norm hidden of each step (in
    the weights' dtype: bf16, or float32 for the float32 evaluation)."""
    from oracle import reference_path as ref
    dt = weights["embed"].dtype
    inv = ref.rope_inv_freq(c.head_dim, c.theta)
    cs = ref.cos_sin_cache(inv, c.max_seq)
    nblk = c.max_seq // c.block
    kc = [torch.zeros(nblk, c.block, c.kv_heads, c.head_dim, dtype=dt) for _ in range(c.layers)]
    vc = [torch.zeros(nblk, c.block, c.kv_heads, c.head_dim, dtype=dt) for _ in range(c.layers)]
    bt = torch.arange(nblk, dtype=torch.int32).reshape(1, nblk)
    seqlen = 0
    outs = []
    kvd = c.kv_heads * c.head_dim
    dims_qkv = [c.hidden, kvd, kvd]
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
