"""CPU oracle: a torch-CPU restatement of SwarmLoRA's hot path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker (or as the
timed CPU baseline).  The product path (swarmlora_amd) never imports it.

Every function restates, in plain torch-CPU ops on bf16 tensors, the
arithmetic of the reference file:line it cites, in the reference's operation
order (so its bf16 roundings are the reference's).  The reference's C++/CUDA
extensions cannot be built here (they need the CUDA toolkit, libtorch-CUDA and
a GPU: /root/reference/setup.py:2-22), and its worker modules import vllm,
which is absent, so nothing from the reference is imported or run.

Third-party arithmetic the reference delegates to (vllm 0.6.6.post1
flash_attn_with_kvcache / rotary_embedding, torch 2.5.1 cuBLAS matmul,
transformers 4.57.3 LlamaRotaryEmbedding) is restated from its published
definition: textbook causal softmax attention, NeoX rotation, x @ W^T with
fp32 accumulation.  How each function is pinned is listed in the tests
(tests/test_oracle.py); none is "parity unpinned".
"""

from typing import Dict, List, Optional, Sequence, Tuple

import math
import torch

BF16 = torch.bfloat16

# op codes, src/cpp_extensions/common/ipc_types.h:19-25
OP_O_PROJ = 3
OP_DOWN_PROJ = 6
OP_QKV_FUSED = 9
OP_GATE_UP_FUSED = 10


# ----------------------------------------------------------- round: gather --
def gather(slot_inputs: Sequence[torch.Tensor], rows: Sequence[int]) -> torch.Tensor:
    """torch::cat of from_blob views [t_i, D] in command (ring-arrival) order,
    ext_aggregator.cpp:545-551."""
    views = [s.reshape(-1, s.shape[-1])[: int(t)] for s, t in zip(slot_inputs, rows)]
    return torch.cat(views, 0)


def scatter(y: torch.Tensor, rows: Sequence[int]) -> List[torch.Tensor]:
    """Per-slot from_blob(out).copy_(output.narrow(0, offset, t_i)),
    ext_aggregator.cpp:564-570: slot i receives rows [off_i, off_i + t_i) at
    offset 0 of its output buffer."""
    outs, off = [], 0
    for t in rows:
        outs.append(y.narrow(0, off, int(t)).clone())
        off += int(t)
    return outs


def base_gemm(x: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """torch::matmul_out(out, x, W.t()) (+ out.add_(bias)) in bf16,
    ext_aggregator.cpp:562, :576-580, :598, :612-616."""
    out = torch.matmul(x, w.t())
    if bias is not None and bias.numel() > 0:
        out = out + bias
    return out


def fuse_layer_weights(q, k, v, gate, up):
    """init_aggregator_layer: qkv = cat(q, k, v, dim 0), gate_up = cat(gate,
    up, dim 0), ext_aggregator.cpp:366-370."""
    return torch.cat([q, k, v], 0), torch.cat([gate, up], 0)


def execute_round(slot_inputs, rows, w, bias=None) -> List[torch.Tensor]:
    """execute_batched_gemm_slots for N slots: gather -> GEMM -> scatter
    (ext_aggregator.cpp:526-625; the N==1 path :491-524 computes the same
    product on the slot buffer directly)."""
    x = gather(slot_inputs, rows)
    y = base_gemm(x, w, bias)
    return scatter(y, rows)


# ----------------------------------------------------------------- LoRA -----
def fused_lora_weights(modules: Sequence[Optional[Tuple[torch.Tensor, torch.Tensor, float]]],
                       out_dims: Sequence[int], dtype=None):
    """FusedLoRA.__init__, model_builder.py:217-256.  modules[i] is
    (lora_A [r, in], lora_B [out_i, r], scaling) or None.
    fused_A = cat_i(A_i^T * s_i) (scale folded in bf16); fused_B is
    block-diagonal [n*r, sum(out_dims)]; missing modules are zero blocks of the
    first valid module's rank."""
    valid = [m for m in modules if m is not None]
    if not valid:
        return None, None
    rank = valid[0][0].shape[0]
    in_features = valid[0][0].shape[1]
    dtype = valid[0][0].dtype if dtype is None else dtype
    a_list, b_list = [], []
    for i, m in enumerate(modules):
        if m is not None:
            A, B, s = m
            a_list.append(A.t() * s)
            b_list.append(B.t())
        else:
            a_list.append(torch.zeros(in_features, rank, dtype=dtype))
            b_list.append(torch.zeros(rank, out_dims[i], dtype=dtype))
    fused_A = torch.cat(a_list, dim=1)
    r = a_list[0].shape[1]
    fused_B = torch.zeros(r * len(modules), sum(out_dims), dtype=dtype)
    col = 0
    for i, B in enumerate(b_list):
        fused_B[i * r:(i + 1) * r, col:col + out_dims[i]] = B
        col += out_dims[i]
    return fused_A, fused_B


def fused_lora_forward(x: torch.Tensor, fused_A, fused_B, out_dims) -> List[torch.Tensor]:
    """FusedLoRA.forward: (dropout(x) @ fused_A) @ fused_B, split(out_dims);
    dropout is Identity.  model_builder.py:258-262.  The [t, n*r]
    intermediate is rounded to bf16 by the first matmul."""
    delta = (x @ fused_A) @ fused_B
    return list(delta.split(list(out_dims), dim=-1))


def remote_lora_delta(x: torch.Tensor, A: torch.Tensor, B: torch.Tensor, scaling: float) -> torch.Tensor:
    """SyncRemoteLoRALinear delta: lora_B(lora_A(dropout(x))) * scaling,
    worker_sync.py:305 (O) and :375 (Down); A [r, in], B [out, r]."""
    return ((x @ A.t()) @ B.t()) * scaling


def qkv_get(base_qkv: torch.Tensor, dims, deltas) -> List[torch.Tensor]:
    """get_outputs_slot split + `q + q_delta` etc., ext_unified_barrier.cpp:
    321-324 and worker_sync.py:276-284."""
    parts = list(base_qkv.split(list(dims), dim=-1))
    if deltas is None:
        return parts
    return [p + d if d is not None else p for p, d in zip(parts, deltas)]


def o_down_get(base: torch.Tensor, residual: torch.Tensor, delta: Optional[torch.Tensor]) -> torch.Tensor:
    """h = residual + (o + delta), worker_sync.py:314-319 and :383-389."""
    r = base + delta if delta is not None else base
    return residual + r


def round_with_lora(op: int, slot_inputs, rows, w, adapters, dims):
    """One round as the reference computes it end to end for every slot:
    aggregator gather/GEMM/scatter, then each worker adds its own delta.
    adapters[i] is None or a list (per column block) of (A [r, in], B [out, r],
    s).  Returns per-slot outputs concatenated over the column blocks (what the
    fused round writes to each slot)."""
    base = execute_round(slot_inputs, rows, w)
    outs = []
    for i, (b, t) in enumerate(zip(base, rows)):
        x = slot_inputs[i].reshape(-1, slot_inputs[i].shape[-1])[: int(t)]
        ad = adapters[i] if adapters is not None else None
        if ad is None:
            outs.append(b)
            continue
        if op in (OP_QKV_FUSED, OP_GATE_UP_FUSED):
            fA, fB = fused_lora_weights(ad, dims)
            deltas = fused_lora_forward(x, fA, fB, dims)
            outs.append(torch.cat(qkv_get(b, dims, deltas), dim=-1))
        else:
            A, B, s = ad[0]
            outs.append(b + remote_lora_delta(x, A, B, s))
    return outs


# ------------------------------------------------------------ embed round --
def embed_round(slot_ids: Sequence[torch.Tensor], table: torch.Tensor) -> List[torch.Tensor]:
    """execute_batched_embed_slots, ext_aggregator.cpp:630-706: the int64 token
    ids of every slot, concatenated in command order, clamped to [0, vocab-1]
    (:663, :694), looked up with torch::embedding and copied back to each
    slot's output rows [t_i, hidden]."""
    counts = [int(t.numel()) for t in slot_ids]
    ids = torch.cat([t.reshape(-1) for t in slot_ids]).clamp(0, table.shape[0] - 1)
    emb = torch.nn.functional.embedding(ids, table)
    return scatter(emb, counts)


# ------------------------------------------------------- paged KV cache -----
class PagedKVCacheRef:
    """Block bookkeeping of PagedKVCache, paged_attention.py:7-118 (metadata
    only; the pages themselves are plain tensors held by the caller)."""

    def __init__(self, block_size: int, max_slots: int, max_seq_len: int):
        self.block_size = block_size
        self.max_blocks_per_seq = (max_seq_len + block_size - 1) // block_size
        self.num_blocks = max_slots * self.max_blocks_per_seq
        self.free_blocks = list(range(self.num_blocks - 1, -1, -1))
        self.slot_block_tables: Dict[int, List[int]] = {}
        self.slot_seq_lens: Dict[int, int] = {}

    def allocate_blocks(self, slot_id, n):
        if len(self.free_blocks) < n:
            raise RuntimeError(f"PagedKVCache: need {n} blocks but only {len(self.free_blocks)} free")
        blocks = [self.free_blocks.pop() for _ in range(n)]
        if slot_id in self.slot_block_tables:
            self.slot_block_tables[slot_id].extend(blocks)
        else:
            self.slot_block_tables[slot_id] = blocks
            self.slot_seq_lens[slot_id] = 0

    def ensure_blocks_for_length(self, slot_id, needed_len):
        need = (needed_len + self.block_size - 1) // self.block_size
        cur = len(self.slot_block_tables.get(slot_id, []))
        if need > cur:
            self.allocate_blocks(slot_id, need - cur)

    def free_slot(self, slot_id):
        blocks = self.slot_block_tables.pop(slot_id, [])
        self.free_blocks.extend(blocks)
        self.slot_seq_lens.pop(slot_id, None)
        return blocks


# ------------------------------------------------------------- RoPE / attn --
def rope_inv_freq(head_dim: int, theta: float, rope_scaling: dict = None) -> torch.Tensor:
    """RoPE inverse frequencies of HF LlamaRotaryEmbedding, which
    model_builder.py:293-296 builds from the model config: theta^(-2i/d), and
    with rope_scaling {"rope_type": "llama3", "factor", "low_freq_factor",
    "high_freq_factor", "original_max_position_embeddings"} (Llama 3.1) the
    published Llama 3.1 frequency remap: wavelengths 2*pi/f longer than
    L/low_freq_factor are divided by factor, shorter than L/high_freq_factor
    kept, and in between interpolated linearly in L/wavelength between f/factor
    and f (L = original_max_position_embeddings)."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    if not rope_scaling:
        return inv
    kind = rope_scaling.get("rope_type", rope_scaling.get("type"))
    if kind == "default":
        return inv
    if kind != "llama3":
        raise ValueError(f"rope_scaling type {kind!r} is not restated here")
    factor = float(rope_scaling["factor"])
    lo, hi = float(rope_scaling["low_freq_factor"]), float(rope_scaling["high_freq_factor"])
    L = float(rope_scaling["original_max_position_embeddings"])
    out = []
    for f in inv.tolist():
        wavelen = 2 * math.pi / f
        if wavelen < L / hi:
            out.append(f)
        elif wavelen > L / lo:
            out.append(f / factor)
        else:
            smooth = (L / wavelen - lo) / (hi - lo)
            out.append((1 - smooth) * f / factor + smooth * f)
    return torch.tensor(out, dtype=torch.float32)


def cos_sin_cache(inv_freq: torch.Tensor, max_seq_len: int, dtype=BF16) -> torch.Tensor:
    """build_vllm_cos_sin_cache, paged_attention.py:131-142: outer(arange fp32,
    inv_freq) -> cat(cos, sin) cast to bf16, [max_seq_len, head_dim]."""
    t = torch.arange(max_seq_len, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq.float())
    return torch.cat([freqs.cos().to(dtype), freqs.sin().to(dtype)], dim=-1)


def rope_neox(x: torch.Tensor, positions: torch.Tensor, cos_sin: torch.Tensor) -> torch.Tensor:
    """NeoX rotation (is_neox=True) of x [ntok, heads, d] at positions [ntok]
    with the bf16 cos|sin cache, worker_sync.py:190-193.  Computed in fp32 and
    rounded once."""
    d = x.shape[-1]
    half = d // 2
    cs = cos_sin[positions.long()].float()
    c = cs[:, :half].unsqueeze(1)
    s = cs[:, half:].unsqueeze(1)
    xf = x.float()
    x1, x2 = xf[..., :half], xf[..., half:]
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1).to(x.dtype)


def paged_attention(q, k_new, v_new, k_cache, v_cache, block_table, cache_seqlens, positions, cos_sin,
                    scale, rope=True):
    """batch_flash_attention, worker_sync.py:169-205: RoPE q/k at positions,
    append k/v into the pages at cache_seqlens[s] + i (flash_attn_with_kvcache
    k/v arguments), then causal GQA attention over cache_seqlens[s] + i + 1
    keys with softmax_scale.  Textbook softmax in fp32.

    q [nseq, L, hq, d]; k_new/v_new [nseq, L, hkv, d]; caches
    [num_blocks, bs, hkv, d] are updated IN PLACE (as flash_attn does).
    Returns (out [nseq, L, hq*d] bf16, q_rot, k_rot)."""
    nseq, L, hq, d = q.shape
    hkv = k_new.shape[2]
    bs = k_cache.shape[1]
    G = hq // hkv
    if rope:
        qr = rope_neox(q.reshape(nseq * L, hq, d), positions, cos_sin).reshape(q.shape)
        kr = rope_neox(k_new.reshape(nseq * L, hkv, d), positions, cos_sin).reshape(k_new.shape)
    else:
        qr, kr = q.clone(), k_new.clone()
    for s in range(nseq):
        for i in range(L):
            p = int(cache_seqlens[s]) + i
            blk = int(block_table[s, p // bs])
            k_cache[blk, p % bs] = kr[s, i]
            v_cache[blk, p % bs] = v_new[s, i]
    out = torch.empty(nseq, L, hq * d, dtype=q.dtype)
    for s in range(nseq):
        ctx_max = int(cache_seqlens[s]) + L
        nblk = (ctx_max + bs - 1) // bs
        blocks = block_table[s, :nblk].long()
        K = k_cache[blocks].reshape(nblk * bs, hkv, d)[:ctx_max].float()
        V = v_cache[blocks].reshape(nblk * bs, hkv, d)[:ctx_max].float()
        for i in range(L):
            ctx = int(cache_seqlens[s]) + i + 1
            qs = qr[s, i].float().reshape(hkv, G, d)
            Kc = K[:ctx].permute(1, 0, 2)          # [hkv, ctx, d]
            Vc = V[:ctx].permute(1, 0, 2)
            sc = torch.einsum("hgd,hcd->hgc", qs, Kc) * scale
            p_ = torch.softmax(sc, dim=-1)
            o = torch.einsum("hgc,hcd->hgd", p_, Vc)
            out[s, i] = o.reshape(hq * d).to(q.dtype)
    return out, qr, kr


# ------------------------------------------------------------- layer step ---
def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """LlamaRMSNorm (transformers 4.57): fp32 variance, x * rsqrt(var + eps),
    cast back, times weight (worker_sync.py:1344-1350 calls it per layer)."""
    xf = x.float()
    var = xf.pow(2).mean(-1, keepdim=True)
    return weight * (xf * torch.rsqrt(var + eps)).to(x.dtype)


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """F.silu(gate) * up in bf16, worker_sync.py:158, :1397."""
    return torch.nn.functional.silu(gate) * up


# ------------------------------------------------------- batched decode step --
def decode_step(cfg, weights, adapters, k_caches, v_caches, block_table, seqlens, ids, cos_sin,
                layers: Optional[int] = None):
    """One token for W workers, in the order of the reference's per-token
    driver (worker_sync.py:1337-1420) with the aggregator's batched rounds
    (ext_aggregator.cpp:545-621: cat of the W token rows, x @ W^T, per-worker
    rows back): embed, per layer input RMSNorm -> QKV round + FusedLoRA delta
    -> RoPE/append/attention -> O round + delta + residual -> post RMSNorm ->
    Gate+Up round + FusedLoRA delta -> SiLU*up -> Down round + delta +
    residual; final norm; LM head (greedy uses argmax of these logits).

    cfg: hidden, heads, kv_heads, head_dim, inter, eps, scale (LoRA scaling).
    weights: {"layers": [{q,k,v,o,gate,up,down,input_norm,post_norm}],
    "embed", "lm_head", "final_norm"} (CPU bf16).  adapters[w]: {layer: {proj:
    (A [r, in], B [out, r])}} or None.  k/v_caches: per-layer page pools
    [num_blocks, bs, kv_heads, head_dim], appended IN PLACE.  seqlens: int32
    [W] context before the step; ids: int64 [W].  layers limits the layer
    count (a partial step, for timing samples).
    Returns (final-norm hidden [W, hidden], logits [W, vocab])."""
    W = ids.numel()
    hq, hkv, hd = cfg.heads, cfg.kv_heads, cfg.head_dim
    kvd = hkv * hd
    dims_qkv = [hq * hd, kvd, kvd]
    dims_gu = [cfg.inter, cfg.inter]
    h = weights["embed"][ids.reshape(-1)]                       # [W, hidden]
    pos = seqlens.long()
    n_layers = len(weights["layers"]) if layers is None else layers
    for li in range(n_layers):
        w = weights["layers"][li]
        res = h
        x = rms_norm(h, w["input_norm"], cfg.eps)
        Wqkv, Wgu = fuse_layer_weights(w["q"], w["k"], w["v"], w["gate"], w["up"])
        base = base_gemm(x, Wqkv)
        q, k, v = [], [], []
        for s in range(W):
            ad = adapters[s][li] if adapters[s] is not None else None
            deltas = None
            if ad is not None:
                fA, fB = fused_lora_weights([(*ad[p], cfg.scale) for p in ("q", "k", "v")], dims_qkv)
                deltas = fused_lora_forward(x[s:s + 1], fA, fB, dims_qkv)
            qs, ks, vs = qkv_get(base[s:s + 1], dims_qkv, deltas)
            q.append(qs), k.append(ks), v.append(vs)
        q = torch.cat(q).reshape(W, 1, hq, hd)
        k = torch.cat(k).reshape(W, 1, hkv, hd)
        v = torch.cat(v).reshape(W, 1, hkv, hd)
        attn, _, _ = paged_attention(q, k, v, k_caches[li], v_caches[li], block_table, seqlens, pos, cos_sin,
                                     1.0 / math.sqrt(hd))
        xa = attn.reshape(W, hq * hd)
        o = base_gemm(xa, w["o"])
        h = torch.cat([o_down_get(o[s:s + 1], res[s:s + 1],
                                  remote_lora_delta(xa[s:s + 1], *adapters[s][li]["o"], cfg.scale)
                                  if adapters[s] is not None else None) for s in range(W)])
        res = h
        x = rms_norm(h, w["post_norm"], cfg.eps)
        gu = base_gemm(x, Wgu)
        m = []
        for s in range(W):
            deltas = None
            if adapters[s] is not None:
                ad = adapters[s][li]
                fA, fB = fused_lora_weights([(*ad[p], cfg.scale) for p in ("gate", "up")], dims_gu)
                deltas = fused_lora_forward(x[s:s + 1], fA, fB, dims_gu)
            g, u = qkv_get(gu[s:s + 1], dims_gu, deltas)
            m.append(silu_mul(g, u))
        m = torch.cat(m)
        d = base_gemm(m, w["down"])
        h = torch.cat([o_down_get(d[s:s + 1], res[s:s + 1],
                                  remote_lora_delta(m[s:s + 1], *adapters[s][li]["down"], cfg.scale)
                                  if adapters[s] is not None else None) for s in range(W)])
    hn = rms_norm(h, weights["final_norm"], cfg.eps)
    logits = base_gemm(hn, weights["lm_head"])
    return hn, logits
