"""One batched decode step for W workers on one GPU, as a single HIP stream.

What one token of SwarmLoRA's serving loop does on the GPU, in order: the
embed round, then per layer input RMSNorm -> fused-QKV round -> RoPE + KV
append + paged attention -> O round -> residual add + post RMSNorm ->
Gate+Up round -> SiLU*up -> Down round -> residual add, then the final norm
and the LM-head round with greedy sampling (reference per-token driver
src/worker/worker_sync.py:1274-1425, aggregator op sequence
src/cpp_extensions/ext_aggregator.cpp:1095-1199).

Here every worker is a slot of the aggregator's pool in this process: the
four projection rounds run through the aggregator runtime
(swl_agg_execute_round over the slots' buffers, LoRA deltas of each worker's
pooled adapter added in the round's epilogue), and the worker-side work reads
and writes the same slot buffers in place (row-mode attention writes the O
round's input rows, SiLU*up writes the Down round's input rows, RMSNorm adds
the round's output rows into the residual stream and writes the next round's
input rows).  The cross-process barrier of the multi-process runtime is
replaced by stream order, so the whole step can be captured as one HIP graph.
"""

import ctypes
from dataclasses import dataclass
from typing import Dict, List, Optional

import torch

from . import _lib
from . import ext_aggregator as agg
from . import ops
from .worker.paged_attention import PagedKVCache

BF16 = torch.bfloat16

PROJ = ("q", "k", "v", "o", "gate", "up", "down")


@dataclass
class DecodeShape:
    """Llama-3.1-8B shape by default (hidden 4096, 32 q / 8 kv heads of 128,
    intermediate 14336, vocabulary 128256, 32 layers)."""
    layers: int = 32
    hidden: int = 4096
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    inter: int = 14336
    vocab: int = 128256
    eps: float = 1e-5
    theta: float = 500000.0
    block_size: int = 16
    rank: int = 16
    scale: float = 2.0

    @property
    def qkv(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    def proj_dims(self) -> Dict[str, tuple]:
        """(in, out) of every projection."""
        h, kv, i = self.hidden, self.kv_heads * self.head_dim, self.inter
        return {"q": (h, h), "k": (h, kv), "v": (h, kv), "o": (h, h), "gate": (h, i), "up": (h, i), "down": (i, h)}

    def step_bytes(self, ctx_lens: List[int], n_adapters: int) -> int:
        """Algorithmic HBM bytes of one step: every weight once, each distinct
        adapter's A and B once, the KV context once, the LM head once."""
        dims = self.proj_dims()
        base = sum(i * o for i, o in dims.values()) * 2 * self.layers
        lora = sum(self.rank * (i + o) for i, o in dims.values()) * 2 * self.layers * n_adapters
        kv = sum(ctx_lens) * 2 * self.kv_heads * self.head_dim * 2 * self.layers
        return base + lora + kv + self.vocab * self.hidden * 2


def synthetic_weights(shape: DecodeShape, device, seed: int = 0, std: float = 0.02) -> dict:
    """Random-init weights on `device`: projections, embedding and LM head
    ~N(0, std), RMSNorm weights 1."""
    g = torch.Generator(device=device).manual_seed(seed)

    def rn(*s):
        return (torch.randn(*s, generator=g, device=device, dtype=torch.float32) * std).to(BF16)

    dims = shape.proj_dims()
    layers = []
    for _ in range(shape.layers):
        w = {p: rn(o, i) for p, (i, o) in dims.items()}
        w["input_norm"] = torch.ones(shape.hidden, dtype=BF16, device=device)
        w["post_norm"] = torch.ones(shape.hidden, dtype=BF16, device=device)
        layers.append(w)
    return {"layers": layers, "embed": rn(shape.vocab, shape.hidden), "lm_head": rn(shape.vocab, shape.hidden),
            "final_norm": torch.ones(shape.hidden, dtype=BF16, device=device)}


def synthetic_adapter(shape: DecodeShape, device, seed: int, std: float = 0.02) -> dict:
    """{layer: {proj: (A [rank, in], B [out, rank])}}, ~N(0, std); all of an
    adapter's matrices are views of one buffer filled by a single draw."""
    g = torch.Generator(device=device).manual_seed(seed)
    dims = shape.proj_dims()
    per_layer = sum(shape.rank * (i + o) for i, o in dims.values())
    flat = (torch.randn(shape.layers * per_layer, generator=g, device=device) * std).to(BF16)
    out, off = {}, 0
    for li in range(shape.layers):
        out[li] = {}
        for p, (i, o) in dims.items():
            a = flat[off:off + shape.rank * i].view(shape.rank, i)
            off += shape.rank * i
            b = flat[off:off + o * shape.rank].view(o, shape.rank)
            off += o * shape.rank
            out[li][p] = (a, b)
    return out


class BatchedDecoder:
    """W one-token decode slots over a shared slot pool and paged KV cache.

    weights: as returned by synthetic_weights (tensors may live on the CPU;
    they are copied to `device`).  adapters[w]: as returned by
    synthetic_adapter, or None for a worker without an adapter.
    ctx_lens[w]: tokens already in worker w's KV pages; kv_fill(layer, k_cache,
    v_cache, block_tables) fills the pages (default: leave them zero).
    Capacity for `max_new` generated tokens is reserved up front.
    packed (fused step only): projection and LM-head weights kept in the
    fragment-tile layout (ops.PackedWeight) instead of row-major.
    whole_k (packed step only, at most 32 workers): the LM head runs as a
    whole-K round (w_layout 2: one launch, no K-slice partials; 206 us
    against 248 for the K-sliced round at 28 workers); the projection rounds
    are K-sliced (whole-K rounds measured slower for them).
    """

    def __init__(self, shape: DecodeShape, weights: dict, adapters: List[Optional[dict]], ctx_lens: List[int],
                 first_ids: List[int], device, max_new: int = 64, kv_fill=None, fused: bool = True,
                 packed: bool = True, whole_k: bool = True):
        self.shape = s = shape
        self.device = dev = torch.device(device)
        self.W = W = len(ctx_lens)
        if not 1 <= W <= ops.RowSet.MAX_ROWS:
            raise ValueError(f"1..{ops.RowSet.MAX_ROWS} workers")
        if len(adapters) != W or len(first_ids) != W:
            raise ValueError("one adapter entry and one first token per worker")
        self.max_new = max_new
        self.steps_done = 0
        self.graph = None
        self.fused = fused
        self.packed = packed and fused
        self.whole_k = bool(whole_k) and self.packed and W <= 32
        if fused:
            self._init_fused(weights, adapters, ctx_lens, first_ids, kv_fill)
            return
        dev_index = dev.index if dev.index is not None else torch.cuda.current_device()

        # ---- slot pool: one slot per worker (1 token per step)
        agg.init_slot_pool(W, dev_index, s.hidden, s.inter, s.kv_heads, s.head_dim, 1, 2)
        self.slot_ids, self.worker_ids = [], []
        for w in range(W):
            info = agg.claim_slot(w)
            self.slot_ids.append(info["slot_id"])
            self.worker_ids.append(w)
        views = [agg.slot_tensors(sid) for sid in self.slot_ids]
        self.slot_in = [v[0] for v in views]
        self.slot_out = [v[1] for v in views]

        # ---- weights (the aggregator fuses q|k|v and gate|up into its own copies)
        agg.init_aggregator_begin(s.layers, dev_index)
        self.norms = []
        for li, lw in enumerate(weights["layers"]):
            t = {k: v.to(dev) for k, v in lw.items()}
            agg.init_aggregator_layer(li, t["q"], t["k"], t["v"], t["o"], None, t["gate"], t["up"], t["down"], None)
            self.norms.append((t["input_norm"].contiguous(), t["post_norm"].contiguous()))
            del t
        agg.init_aggregator_finalize()
        self.embed = weights["embed"].to(dev).contiguous()
        self.lm_head = weights["lm_head"].to(dev).contiguous()
        self.final_norm = weights["final_norm"].to(dev).contiguous()
        agg.init_embed_lm_head_weights(self.embed, self.lm_head)

        # ---- adapters: pooled, adapter id = worker index
        agg.clear_adapters()
        self.adapter_ids = []
        for w, ad in enumerate(adapters):
            if ad is None:
                self.adapter_ids.append(-1)
                continue
            self.adapter_ids.append(w)
            for li in range(s.layers):
                a = ad[li]
                for op, projs in ((agg.OP_QKV_FUSED, ("q", "k", "v")), (agg.OP_O_PROJ, ("o",)),
                                  (agg.OP_GATE_UP_FUSED, ("gate", "up")), (agg.OP_DOWN_PROJ, ("down",))):
                    A = torch.cat([a[p][0].to(dev) for p in projs], 0).contiguous()
                    Bs = [a[p][1].to(dev).contiguous() for p in projs]
                    agg.register_adapter(w, li, op, A, Bs, s.scale)

        # ---- paged KV: the reference keeps one cache per worker; here one
        # pool of pages with a block table per worker
        self._init_kv(ctx_lens, kv_fill)

        # ---- per-step state
        self.ids = torch.tensor(first_ids, dtype=torch.int64, device=dev).reshape(W, 1)
        self.h = torch.zeros(W, s.hidden, dtype=BF16, device=dev)        # residual stream
        self.lm_in = torch.zeros(W, s.hidden, dtype=BF16, device=dev)    # final-norm output
        self.logits = torch.zeros(W, s.vocab, dtype=BF16, device=dev)
        self.rows_in_h = ops.RowSet([t[:s.hidden] for t in self.slot_in], s.hidden)
        self.rows_in_i = ops.RowSet([t[:s.inter] for t in self.slot_in], s.inter)
        self.rows_out_h = ops.RowSet([t[:s.hidden] for t in self.slot_out], s.hidden)
        self.rows_out_qkv = ops.RowSet([t[:s.qkv] for t in self.slot_out], s.qkv)
        self.rows_out_gu = ops.RowSet([t[:2 * s.inter] for t in self.slot_out], 2 * s.inter)
        self.rows_lm = ops.RowSet([self.lm_in[w] for w in range(W)], s.hidden)
        self._ids_rows = [self.ids[w] for w in range(W)]
        self._h_rows = [self.h[w:w + 1] for w in range(W)]
        self._round_args = ((ctypes.c_int32 * W)(*self.slot_ids), (ctypes.c_int32 * W)(*self.worker_ids),
                            (ctypes.c_int64 * W)(*([1] * W)), (ctypes.c_int32 * W)(*self.adapter_ids))
        self._scale = 1.0 / (s.head_dim ** 0.5)

    def _init_kv(self, ctx_lens, kv_fill):
        s, dev, W = self.shape, self.device, self.W
        self.kv = PagedKVCache(s.layers, s.kv_heads, s.head_dim, s.block_size, W, max(ctx_lens) + self.max_new, dev,
                               BF16)
        for w, c in enumerate(ctx_lens):
            self.kv.ensure_blocks_for_length(w, c + self.max_new)
            self.kv.slot_seq_lens[w] = c
        self.block_tables = self.kv.get_block_table_tensor(list(range(W)))
        if kv_fill is not None:
            for li in range(s.layers):
                kv_fill(li, self.kv.key_caches[li], self.kv.value_caches[li], self.block_tables)
        self.seqlens = self.kv.get_seq_lens_tensor(list(range(W)))
        self.positions = torch.zeros(W, dtype=torch.int64, device=dev)
        from .worker.paged_attention import RotaryInvFreq, build_vllm_cos_sin_cache
        self.cos_sin = build_vllm_cos_sin_cache(RotaryInvFreq(s.head_dim, s.theta), self.kv.max_blocks_per_seq *
                                                s.block_size, dev, BF16)

    def _init_fused(self, weights, adapters, ctx_lens, first_ids, kv_fill):
        """In-process step over explicit token rows with the round fusions
        (swl_round_fusion): the input RMSNorm applied while the round stages
        its activation rows, RoPE and the KV append in the QKV round's
        epilogue, the residual adds in the O and Down epilogues and SiLU*up in
        the Gate+Up epilogue."""
        s, dev, W = self.shape, self.device, self.W
        self.layers_w = []
        self.norms = []
        # the whole-K LM head: K a multiple of 256 up to 4096, n a multiple of
        # 16 (measured at 8B widths, 28 workers, in the captured step: 206 us
        # against 248 for split + epilogue; the projection rounds are faster
        # K-sliced at every row count from 1 to 28: with cold weights one
        # tile per CU in flight streams slower, and every CU loads all token
        # rows, more bytes than its share of the O / QKV weights)
        self.wk = {"qkv": False, "o": False, "gu": False, "down": False,
                   "lm": self.whole_k and s.hidden % 256 == 0 and s.hidden <= 4096 and s.vocab % 16 == 0}

        def keep(t, g):
            return ops.pack_weight(t) if self.packed else t

        for lw in weights["layers"]:
            t = {k: v.to(dev) for k, v in lw.items()}
            self.layers_w.append({
                "qkv": keep(torch.cat([t["q"], t["k"], t["v"]], 0).contiguous(), "qkv"),
                "o": keep(t["o"].contiguous(), "o"),
                "gu": keep(torch.cat([t["gate"], t["up"]], 0).contiguous(), "gu"),
                "down": keep(t["down"].contiguous(), "down"),
            })
            self.norms.append((t["input_norm"].contiguous(), t["post_norm"].contiguous()))
            del t
        self.embed = weights["embed"].to(dev).contiguous()
        self.lm_head = keep(weights["lm_head"].to(dev).contiguous(), "lm")
        self.final_norm = weights["final_norm"].to(dev).contiguous()

        # adapters: one table entry per (worker, layer, fused projection);
        # the K-sliced rounds of the packed step stream the stacked lora_A as
        # fragment tiles like their weights (row-major A rows, 64-byte pieces
        # of 16 rows per load, were the last waves of the QKV and O rounds)
        self.a_packed = {g: self.packed and not self.wk[g] for g in ("qkv", "o", "gu", "down")}
        self.table = ops.LoraTable(dev)
        groups = (("qkv", ("q", "k", "v")), ("o", ("o",)), ("gu", ("gate", "up")), ("down", ("down",)))
        self.seg_lora = [{g: [-1] * W for g, _ in groups} for _ in range(s.layers)]
        for w, ad in enumerate(adapters):
            if ad is None:
                continue
            for li in range(s.layers):
                for g, projs in groups:
                    A = torch.cat([ad[li][p][0].to(dev) for p in projs], 0).contiguous()
                    Bs = [ad[li][p][1].to(dev).contiguous() for p in projs]
                    if self.a_packed[g]:
                        A = ops.pack_weight(A)
                    self.seg_lora[li][g][w] = self.table.add(A, Bs, s.rank, s.scale)
        has_lora = any(ad is not None for ad in adapters)
        blk = {"qkv": [s.hidden, s.kv_heads * s.head_dim, s.kv_heads * s.head_dim], "o": [s.hidden],
               "gu": [s.inter, s.inter], "down": [s.hidden]}

        self._init_kv(ctx_lens, kv_fill)

        # per-step buffers: one row per worker; partial sums of squares of the
        # residual stream, one per 256 columns (written by the O and Down
        # rounds' epilogues)
        nss_o = nss_d = (s.hidden + 255) // 256
        self.ids = torch.tensor(first_ids, dtype=torch.int64, device=dev).reshape(W, 1)
        self.h = torch.zeros(W, s.hidden, dtype=BF16, device=dev)        # residual stream
        self.x0 = torch.zeros(W, s.hidden, dtype=BF16, device=dev)       # layer 0's normed input
        self.qkv = torch.zeros(W, s.qkv, dtype=BF16, device=dev)
        self.attn = torch.zeros(W, s.heads * s.head_dim, dtype=BF16, device=dev)
        self.act = torch.zeros(W, s.inter, dtype=BF16, device=dev)
        self.logits = torch.zeros(W, s.vocab, dtype=BF16, device=dev)
        self.ss_o = torch.zeros(W, nss_o, dtype=torch.float32, device=dev)
        self.ss_d = torch.zeros(W, nss_d, dtype=torch.float32, device=dev)
        rows = lambda t: [t[w:w + 1] for w in range(W)]  # noqa: E731
        self.rows_x0 = ops.RowSet([self.x0[w] for w in range(W)], s.hidden)
        self.rows_qkv = ops.RowSet([self.qkv[w] for w in range(W)], s.qkv)
        self.rows_attn = ops.RowSet([self.attn[w] for w in range(W)], s.heads * s.head_dim)
        self._ids_rows = [self.ids[w] for w in range(W)]
        self._h_rows = rows(self.h)

        # the 4 rounds of every layer and the LM head, arguments built once
        one = [1] * W
        self._calls = []
        for li in range(s.layers):
            lw, (in_norm, post_norm) = self.layers_w[li], self.norms[li]
            kv = dict(k_cache=self.kv.key_caches[li], v_cache=self.kv.value_caches[li], hq=s.heads, hkv=s.kv_heads,
                      block_table=self.block_tables, cache_seqlens=self.seqlens, positions=self.positions,
                      cos_sin=self.cos_sin)
            wl = {g: (2 if self.wk[g] else 1) if self.packed else 0 for g in self.wk}
            al = {g: 1 if has_lora and self.a_packed[g] else 0 for g in self.a_packed}
            qkv_out = dict(out_mode=3, **kv)
            plan = (
                ("qkv", rows(self.x0) if li == 0 else rows(self.h), rows(self.qkv),
                 ops.round_fusion(w_layout=wl["qkv"], a_layout=al["qkv"], **qkv_out) if li == 0 else
                 ops.round_fusion(norm_weight=in_norm, eps=s.eps, ss_in=self.ss_d, w_layout=wl["qkv"],
                                  a_layout=al["qkv"], **qkv_out)),
                ("o", rows(self.attn), rows(self.h),
                 ops.round_fusion(out_mode=1, ss_out=self.ss_o, w_layout=wl["o"], a_layout=al["o"])),
                ("gu", rows(self.h), rows(self.act),
                 ops.round_fusion(norm_weight=post_norm, eps=s.eps, ss_in=self.ss_o, out_mode=2, w_layout=wl["gu"],
                                  a_layout=al["gu"])),
                ("down", rows(self.act), rows(self.h),
                 ops.round_fusion(out_mode=1, ss_out=self.ss_d, w_layout=wl["down"], a_layout=al["down"])),
            )
            layer_calls = []
            for g, xin, yout, fz in plan:
                args = ops._round_args(xin, yout, one, lw[g], None, self.seg_lora[li][g] if has_lora else None,
                                       self.table if has_lora else None, blk[g] if has_lora else None,
                                       out_div=2 if fz.out_mode == 2 else 1)
                layer_calls.append((args, fz))
            self._calls.append(layer_calls)
        lm_fz = ops.round_fusion(norm_weight=self.final_norm, eps=s.eps, ss_in=self.ss_d,
                                 w_layout=(2 if self.wk["lm"] else 1) if self.packed else 0)
        self._lm_call = (ops._round_args(rows(self.h), rows(self.logits), one, self.lm_head, None, None, None, None),
                         lm_fz)
        self._scale = 1.0 / (s.head_dim ** 0.5)

    @property
    def final_h(self) -> torch.Tensor:
        """The residual stream after the last layer (what the final norm and
        the LM head read): [W, hidden]."""
        return self.h

    def _round_ex(self, call):
        args, fz = call
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(_lib.load().swl_round_ex_bf16(*args, ctypes.byref(fz), st))

    def _body_fused(self):
        s = self.shape
        self.positions.copy_(self.seqlens)
        ops.embed(self._ids_rows, self.embed, self._h_rows)
        ops.rmsnorm_rows(self.h, self.norms[0][0], s.eps, self.rows_x0)
        for li in range(s.layers):
            qkv, o, gu, down = self._calls[li]
            self._round_ex(qkv)
            ops.paged_attention_rows(self.rows_qkv, self.rows_attn, 1, s.heads, s.kv_heads, s.head_dim,
                                     self.kv.key_caches[li], self.kv.value_caches[li], self.block_tables,
                                     self.seqlens, None, None, self._scale, rope=2)
            self._round_ex(o)
            self._round_ex(gu)
            self._round_ex(down)
        self._round_ex(self._lm_call)
        W = self.W
        ops.sample(self.logits, self._ids_rows, [False] * W, [1.0] * W, [0] * W, [1.0] * W, 0)
        self.seqlens.add_(1)

    # ------------------------------------------------------------ one step
    def _round(self, op: int, layer: int):
        s_arr, w_arr, t_arr, a_arr = self._round_args
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(_lib.load().swl_agg_execute_round(op, layer, self.W, s_arr, w_arr, t_arr, a_arr, st))

    def _body(self):
        s = self.shape
        self.positions.copy_(self.seqlens)
        ops.embed(self._ids_rows, self.embed, self._h_rows)
        for li in range(s.layers):
            in_norm, post_norm = self.norms[li]
            ops.rmsnorm_rows(self.h, in_norm, s.eps, self.rows_in_h, add_rows=self.rows_out_h if li else None)
            self._round(agg.OP_QKV_FUSED, li)
            ops.paged_attention_rows(self.rows_out_qkv, self.rows_in_h, 1, s.heads, s.kv_heads, s.head_dim,
                                     self.kv.key_caches[li], self.kv.value_caches[li], self.block_tables,
                                     self.seqlens, self.positions, self.cos_sin, self._scale)
            self._round(agg.OP_O_PROJ, li)
            ops.rmsnorm_rows(self.h, post_norm, s.eps, self.rows_in_h, add_rows=self.rows_out_h)
            self._round(agg.OP_GATE_UP_FUSED, li)
            ops.silu_mul_rows(self.rows_out_gu, self.rows_in_i, s.inter)
            self._round(agg.OP_DOWN_PROJ, li)
        ops.rmsnorm_rows(self.h, self.final_norm, s.eps, self.rows_lm, add_rows=self.rows_out_h)
        ops.gemm(self.lm_in, self.lm_head, out=self.logits)
        W = self.W
        ops.sample(self.logits, self._ids_rows, [False] * W, [1.0] * W, [0] * W, [1.0] * W, 0)
        self.seqlens.add_(1)

    def _check_capacity(self):
        if self.steps_done >= self.max_new:
            raise RuntimeError(f"BatchedDecoder: KV pages reserved for {self.max_new} new tokens are used up")

    def _step_body(self):
        if self.fused:
            self._body_fused()
        else:
            self._body()

    def step_eager(self):
        """Launch one step's kernels on the current stream."""
        self._check_capacity()
        self._step_body()
        self.steps_done += 1

    def capture(self):
        """Capture one step as a HIP graph (call after one eager step, which
        sizes the library's scratch and uploads the adapter table)."""
        if self.steps_done == 0:
            raise RuntimeError("run step_eager() once before capture()")
        # the captured body is not executed; the graph is replayed by step()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._step_body()
        self.graph = g

    def step(self):
        """One decode step: graph replay if captured, else eager."""
        if self.graph is None:
            return self.step_eager()
        self._check_capacity()
        self.graph.replay()
        self.steps_done += 1

    def close(self):
        self.graph = None
        if self.fused:
            return
        for sid, wid in zip(self.slot_ids, self.worker_ids):
            agg.release_slot(sid, wid)
        agg.clear_adapters()
        agg.cleanup_slot_pool()
