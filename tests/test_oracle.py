"""Pins the CPU oracle (oracle/reference_path.py) before it is trusted.

The reference ships no golden vectors, known-answer tests or fixtures for this
path (its repo has no test suite), and none of its code can be built or run
here.  Each oracle function is therefore pinned by checks chosen so that a
plausible mistake (dropped term, wrong sign or index, transposed operand,
wrong rounding order) fails one of them: brute force on tiny inputs, closed
forms, special cases that reduce to textbook routines, and invariants.
"""

import math

import pytest
import torch

from oracle import reference_path as ref
from tests._util import BF16, bits_equal, randn, rel_err


# ------------------------------------------------------------ gather/scatter
def test_gather_matches_bruteforce_rows():
    rows = [2, 0, 3, 1]
    slots = [randn((4, 6), i) for i in range(4)]
    got = ref.gather(slots, rows)
    brute = []
    for s, t in zip(slots, rows):
        for j in range(t):
            brute.append(s[j])
    assert bits_equal(got, torch.stack(brute))


def test_scatter_inverts_gather():
    rows = [3, 1, 0, 2]
    slots = [randn((t + 1, 5), 10 + i)[:t] for i, t in enumerate(rows)]
    back = ref.scatter(ref.gather(slots, rows), rows)
    for a, b in zip(back, slots):
        assert bits_equal(a, b)


def test_round_results_independent_of_arrival_order():
    rows = [1, 3, 2]
    w = randn((24, 32), 0)
    xs = [randn((t, 32), 20 + i) for i, t in enumerate(rows)]
    a = ref.execute_round(xs, rows, w)
    perm = [2, 0, 1]
    b = ref.execute_round([xs[p] for p in perm], [rows[p] for p in perm], w)
    for i, p in enumerate(perm):
        assert bits_equal(b[i], a[p])


def test_embed_round_clamps_and_scatters_bruteforce():
    """Each slot's rows are table rows of its ids clamped to [0, vocab-1]
    (negative ids -> row 0, ids >= vocab -> the last row), in slot order."""
    table = randn((9, 5), 30)
    ids = [torch.tensor([3, -1, 8]), torch.tensor([], dtype=torch.int64), torch.tensor([9, 100, 0, -7])]
    got = ref.embed_round(ids, table)
    assert [g.shape[0] for g in got] == [3, 0, 4]
    for g, t in zip(got, ids):
        for j, v in enumerate(t.tolist()):
            assert bits_equal(g[j], table[min(max(v, 0), 8)])


# -------------------------------------------------------------------- GEMM
def test_base_gemm_one_hot_selects_column():
    w = randn((7, 11), 0)
    x = torch.zeros(3, 11, dtype=BF16)
    x[0, 4] = 1
    x[1, 0] = 1
    x[2, 10] = 1
    y = ref.base_gemm(x, w)
    assert bits_equal(y, w[:, [4, 0, 10]].t().contiguous())


def test_base_gemm_is_x_times_w_transposed():
    x = randn((5, 64), 1)
    w = randn((48, 64), 2, std=0.1)
    y = ref.base_gemm(x, w)
    assert y.shape == (5, 48)
    assert rel_err(y, x.double() @ w.double().t()) < 5e-3
    # a transposed weight must not pass for the real one
    w_sq = randn((64, 64), 3)
    x_sq = randn((5, 64), 4)
    assert rel_err(ref.base_gemm(x_sq, w_sq), x_sq.double() @ w_sq.double()) > 0.1


def test_base_gemm_bias_added_per_output_column():
    x = torch.zeros(2, 8, dtype=BF16)
    w = randn((4, 8), 0)
    b = torch.tensor([1.0, -2.0, 0.5, 3.0], dtype=BF16)
    assert bits_equal(ref.base_gemm(x, w, b), b.expand(2, 4).contiguous())


def test_fuse_layer_weights_row_order():
    q, k, v = randn((8, 4), 0), randn((2, 4), 1), randn((2, 4), 2)
    g, u = randn((6, 4), 3), randn((6, 4), 4)
    qkv, gu = ref.fuse_layer_weights(q, k, v, g, u)
    assert bits_equal(qkv[:8], q) and bits_equal(qkv[8:10], k) and bits_equal(qkv[10:], v)
    assert bits_equal(gu[:6], g) and bits_equal(gu[6:], u)


# -------------------------------------------------------------------- LoRA
def _mods(r, in_dim, out_dims, s, seed=0):
    return [(randn((r, in_dim), seed + 2 * i, std=0.3), randn((o, r), seed + 2 * i + 1, std=0.3), s)
            for i, o in enumerate(out_dims)]


def test_fused_lora_structure_block_diagonal():
    dims = [8, 4, 4]
    mods = _mods(2, 16, dims, 2.0)
    fA, fB = ref.fused_lora_weights(mods, dims)
    assert fA.shape == (16, 6) and fB.shape == (6, 16)
    for i, (A, B, s) in enumerate(mods):
        assert bits_equal(fA[:, 2 * i:2 * i + 2], (A.t() * s))
    col = [0, 8, 12, 16]
    for i in range(3):
        for j in range(3):
            blk = fB[2 * i:2 * i + 2, col[j]:col[j + 1]]
            if i == j:
                assert bits_equal(blk, mods[i][1].t().contiguous())
            else:
                assert float(blk.abs().max()) == 0.0


def test_fused_lora_zero_B_gives_zero_delta():
    dims = [8, 4]
    mods = [(A, torch.zeros_like(B), s) for A, B, s in _mods(4, 16, dims, 2.0)]
    fA, fB = ref.fused_lora_weights(mods, dims)
    for d in ref.fused_lora_forward(randn((3, 16), 9), fA, fB, dims):
        assert float(d.abs().max()) == 0.0


def test_fused_lora_rank1_one_hot_closed_form():
    """x = e_i, A = e_j^T (r=1) => delta = s * A[0, i] * B[:, 0] (exact)."""
    in_dim, dims, s = 8, [6], 2.0
    A = torch.zeros(1, in_dim, dtype=BF16)
    A[0, 3] = 0.5
    B = randn((6, 1), 5)
    fA, fB = ref.fused_lora_weights([(A, B, s)], dims)
    x = torch.zeros(1, in_dim, dtype=BF16)
    x[0, 3] = 1.0
    (d,) = ref.fused_lora_forward(x, fA, fB, dims)
    assert bits_equal(d, (B[:, 0] * 1.0).reshape(1, 6).to(BF16))  # s*0.5 = 1 exactly


def test_fused_lora_blocks_independent():
    dims = [8, 4, 4]
    mods = _mods(4, 16, dims, 2.0, seed=30)
    x = randn((2, 16), 7)
    fA, fB = ref.fused_lora_weights(mods, dims)
    d1 = ref.fused_lora_forward(x, fA, fB, dims)
    mods2 = list(mods)
    A, B, s = mods2[1]
    mods2[1] = (A * 3, B, s)   # perturb k's A only
    fA2, fB2 = ref.fused_lora_weights(mods2, dims)
    d2 = ref.fused_lora_forward(x, fA2, fB2, dims)
    assert bits_equal(d1[0], d2[0]) and bits_equal(d1[2], d2[2])
    assert not bits_equal(d1[1], d2[1])


def test_fused_lora_equals_per_module_delta():
    """Folding the scale into A (FusedLoRA) and applying it last (PEFT) agree
    up to bf16 rounding; both agree with the fp64 closed form."""
    dims = [16, 8]
    mods = _mods(4, 32, dims, 2.0, seed=50)
    x = randn((3, 32), 8)
    fA, fB = ref.fused_lora_weights(mods, dims)
    fused = ref.fused_lora_forward(x, fA, fB, dims)
    for (A, B, s), d in zip(mods, fused):
        per = ref.remote_lora_delta(x, A, B, s)
        exact = (x.double() @ A.double().t() @ B.double().t()) * s
        assert rel_err(d, exact) < 1.5e-2
        assert rel_err(per, exact) < 1.5e-2


def test_missing_module_is_zero_block_with_first_rank():
    dims = [8, 4, 4]
    mods = _mods(2, 16, dims, 1.0)
    mods[1] = None
    fA, fB = ref.fused_lora_weights(mods, dims)
    assert float(fA[:, 2:4].abs().max()) == 0.0
    d = ref.fused_lora_forward(randn((2, 16), 3), fA, fB, dims)
    assert float(d[1].abs().max()) == 0.0


def test_get_adds():
    base = randn((2, 12), 0)
    deltas = [randn((2, 8), 1), None, randn((2, 2), 2)]
    q, k, v = ref.qkv_get(base, [8, 2, 2], deltas)
    assert bits_equal(q, base[:, :8] + deltas[0]) and bits_equal(k, base[:, 8:10])
    res = randn((2, 4), 5)
    o = ref.o_down_get(base[:, :4], res, None)
    assert bits_equal(o, res + base[:, :4])


# ---------------------------------------------------------------- paged KV
def test_paged_kv_allocation_order_and_reuse():
    c = ref.PagedKVCacheRef(block_size=16, max_slots=2, max_seq_len=64)
    assert c.num_blocks == 8 and c.max_blocks_per_seq == 4
    c.ensure_blocks_for_length(0, 17)      # 2 blocks
    c.ensure_blocks_for_length(1, 1)       # 1 block
    c.ensure_blocks_for_length(0, 32)      # still 2
    c.ensure_blocks_for_length(0, 33)      # 3rd block
    assert c.slot_block_tables == {0: [0, 1, 3], 1: [2]}
    freed = c.free_slot(0)
    assert freed == [0, 1, 3]
    c.ensure_blocks_for_length(5, 16)
    assert c.slot_block_tables[5] == [3]   # LIFO: last freed first
    with pytest.raises(RuntimeError):
        c.allocate_blocks(6, 100)


# ------------------------------------------------------------- RoPE / attn
def test_inv_freq_closed_form():
    inv = ref.rope_inv_freq(128, 500000.0)
    for i in (0, 1, 17, 63):
        assert abs(inv[i].item() - 500000.0 ** (-2 * i / 128)) < 1e-9 + 1e-6 * inv[i].item()


def test_cos_sin_row0_and_rope_identity_at_zero():
    cs = ref.cos_sin_cache(ref.rope_inv_freq(128, 10000.0), 8)
    assert bits_equal(cs[0, :64], torch.ones(64, dtype=BF16))
    assert bits_equal(cs[0, 64:], torch.zeros(64, dtype=BF16))
    x = randn((1, 2, 128), 0)
    assert bits_equal(ref.rope_neox(x, torch.tensor([0]), cs), x)


def test_rope_is_complex_rotation_of_half_pairs():
    """NeoX: (x_i, x_{i+64}) rotated by angle p * inv_freq_i."""
    inv = ref.rope_inv_freq(128, 500000.0)
    cs = ref.cos_sin_cache(inv, 64)
    x = randn((3, 1, 128), 1)
    pos = torch.tensor([1, 7, 63])
    y = ref.rope_neox(x, pos, cs).double()
    xd = x.double()
    c = cs[pos].double()[:, None, :64]
    s = cs[pos].double()[:, None, 64:]
    z = torch.complex(xd[..., :64], xd[..., 64:]) * torch.complex(c, s)
    assert rel_err(y, torch.cat([z.real, z.imag], -1)) < 1e-2
    # the GPT-J (interleaved-pair) rotation does not pass for NeoX
    zi = torch.complex(xd[..., 0::2], xd[..., 1::2]) * torch.complex(c, s)
    inter = torch.stack([zi.real, zi.imag], -1).reshape(xd.shape)
    assert rel_err(y, inter) > 0.05


def _attn_tiny(L=1, ctx0=(5, 9), hq=4, hkv=2, bs=4, seed=0, equal_keys=False):
    d = 128
    nseq = len(ctx0)
    maxb = (max(ctx0) + L + bs - 1) // bs
    nb = nseq * maxb
    bt = torch.arange(nb).reshape(nseq, maxb).flip(1).to(torch.int32)
    kc = randn((nb, bs, hkv, d), seed + 1)
    if equal_keys:
        kc[:] = kc[0, 0]
    vc = randn((nb, bs, hkv, d), seed + 2)
    q = randn((nseq, L, hq, d), seed + 3)
    k = kc[0, 0].expand(nseq, L, hkv, d).clone() if equal_keys else randn((nseq, L, hkv, d), seed + 4)
    v = randn((nseq, L, hkv, d), seed + 5)
    sl = torch.tensor(ctx0, dtype=torch.int32)
    return q, k, v, kc, vc, bt, sl


def test_attention_matches_fp64_bruteforce():
    q, k, v, kc, vc, bt, sl = _attn_tiny(L=2)
    kc0, vc0 = kc.clone(), vc.clone()
    out, _, _ = ref.paged_attention(q, k, v, kc, vc, bt, sl, None, None, 0.125, rope=False)
    nseq, L, hq, d = q.shape
    hkv, bs = k.shape[2], kc.shape[1]
    for s in range(nseq):
        toks_k, toks_v = [], []
        for p in range(int(sl[s]) + L):
            if p < int(sl[s]):
                blk = int(bt[s, p // bs])
                toks_k.append(kc0[blk, p % bs])
                toks_v.append(vc0[blk, p % bs])
            else:
                toks_k.append(k[s, p - int(sl[s])])
                toks_v.append(v[s, p - int(sl[s])])
        K = torch.stack(toks_k).double()
        V = torch.stack(toks_v).double()
        for i in range(L):
            ctx = int(sl[s]) + i + 1
            for h in range(hq):
                kh = h // (hq // hkv)
                sc = (K[:ctx, kh] @ q[s, i, h].double()) * 0.125
                p_ = torch.softmax(sc, 0)
                o = p_ @ V[:ctx, kh]
                assert rel_err(out[s, i, h * d:(h + 1) * d], o) < 1e-2


def test_attention_single_key_and_equal_keys():
    q, k, v, kc, vc, bt, sl = _attn_tiny(ctx0=(0,))
    out, _, _ = ref.paged_attention(q, k, v, kc, vc, bt, sl, None, None, 0.1, rope=False)
    for h in range(4):
        assert bits_equal(out[0, 0, h * 128:(h + 1) * 128], v[0, 0, h // 2])
    q, k, v, kc, vc, bt, sl = _attn_tiny(ctx0=(6,), equal_keys=True)
    kc0, vc0 = kc.clone(), vc.clone()
    out, _, _ = ref.paged_attention(q, k, v, kc, vc, bt, sl, None, None, 0.1, rope=False)
    bs = kc.shape[1]
    vals = [vc0[int(bt[0, p // bs]), p % bs] for p in range(6)] + [v[0, 0]]
    mean = torch.stack(vals).double().mean(0)
    for h in range(4):
        assert rel_err(out[0, 0, h * 128:(h + 1) * 128], mean[h // 2]) < 1e-2


def test_attention_gqa_head_mapping():
    """Query head h reads kv head h // (hq / hkv): swapping the kv heads'
    contents must permute the outputs accordingly."""
    q, k, v, kc, vc, bt, sl = _attn_tiny(ctx0=(7,), seed=3)
    out1, _, _ = ref.paged_attention(q, k, v, kc.clone(), vc.clone(), bt, sl, None, None, 0.1, rope=False)
    q2 = q[:, :, [2, 3, 0, 1]].contiguous()
    out2, _, _ = ref.paged_attention(q2, k.flip(2).contiguous(), v.flip(2).contiguous(), kc.flip(2).contiguous(),
                                     vc.flip(2).contiguous(), bt, sl, None, None, 0.1, rope=False)
    o1 = out1.reshape(4, 128)
    o2 = out2.reshape(4, 128)
    assert bits_equal(o2[[2, 3, 0, 1]], o1)


def test_rms_norm_and_silu():
    x = randn((3, 64), 0)
    w = randn((64,), 1)
    y = ref.rms_norm(x, w, 1e-5)
    xd = x.double()
    want = w.double() * (xd / torch.sqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-5))
    assert rel_err(y, want) < 1e-2
    g, u = randn((4, 8), 2), randn((4, 8), 3)
    sm = ref.silu_mul(g, u).double()
    gd = g.double()
    assert rel_err(sm, gd / (1 + torch.exp(-gd)) * u.double()) < 1e-2


# ------------------------------------------------------- batched decode step
_HF_PROJ = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj", "o": "self_attn.o_proj",
            "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}


def _hf_llama(c, wts, ad):
    """transformers' own LlamaForCausalLM (the library the reference's
    worker builds its layers from: RMSNorm, rotary embedding, GQA attention,
    SiLU MLP) in fp32, loaded with the same weights and the LoRA merged
    into them: W + scale * B @ A."""
    transformers = pytest.importorskip("transformers")
    cfg = transformers.LlamaConfig(vocab_size=c.vocab, hidden_size=c.hidden, intermediate_size=c.inter,
                                   num_hidden_layers=c.layers, num_attention_heads=c.heads,
                                   num_key_value_heads=c.kv_heads, head_dim=c.head_dim, rms_norm_eps=c.eps,
                                   rope_theta=c.theta, max_position_embeddings=4096, tie_word_embeddings=False)
    m = transformers.LlamaForCausalLM(cfg).float().eval()
    sd = {"model.embed_tokens.weight": wts["embed"].float(), "lm_head.weight": wts["lm_head"].float(),
          "model.norm.weight": wts["final_norm"].float()}
    for li, lw in enumerate(wts["layers"]):
        for p, name in _HF_PROJ.items():
            wf = lw[p].float()
            if ad is not None:
                A, B = ad[li][p]
                wf = wf + c.scale * (B.float() @ A.float())
            sd[f"model.layers.{li}.{name}.weight"] = wf
        sd[f"model.layers.{li}.input_layernorm.weight"] = lw["input_norm"].float()
        sd[f"model.layers.{li}.post_attention_layernorm.weight"] = lw["post_norm"].float()
    m.load_state_dict(sd, strict=True)
    return m


def test_decode_step_matches_transformers_llama():
    """decode_step run token by token from empty pages (three workers: two
    adapters, one without) equals transformers' LlamaForCausalLM over each
    worker's whole sequence.  Independent of the oracle's own functions: a
    wrong RoPE pairing, GQA head map, norm order, residual, SiLU side or
    page index fails it.  Tolerance: the oracle rounds to bf16 where the
    reference does, the fp32 model does not, so 1.5e-2 normalised max error
    on the logits (measured ~6e-3)."""
    from tests._tiny_model import CFG as c, adapter, base_weights
    wts = base_weights()
    ads = [{li: {p: a[li][_HF_PROJ[p]] for p in _HF_PROJ} for li in a} for a in (adapter(0), adapter(3))]
    ads = [ads[0], None, ads[1]]
    W, T, nb = len(ads), 6, 4
    seqs = torch.randint(0, c.vocab, (W, T), generator=torch.Generator().manual_seed(5))
    kc = [torch.zeros(W * nb, c.block, c.kv_heads, c.head_dim, dtype=BF16) for _ in range(c.layers)]
    vc = [torch.zeros_like(kc[0]) for _ in range(c.layers)]
    bt = torch.randperm(W * nb, generator=torch.Generator().manual_seed(6)).to(torch.int32).reshape(W, nb)
    cs = ref.cos_sin_cache(ref.rope_inv_freq(c.head_dim, c.theta), 64)
    logits = []
    for t in range(T):
        _, lg = ref.decode_step(c, wts, ads, kc, vc, bt, torch.full((W,), t, dtype=torch.int32), seqs[:, t], cs)
        logits.append(lg)
    for w in range(W):
        with torch.no_grad():
            want = _hf_llama(c, wts, ads[w])(seqs[w:w + 1]).logits[0]
        for t in range(T):
            assert rel_err(logits[t][w], want[t]) <= 1.5e-2, (w, t)
            # greedy choice: the oracle's argmax is (near-)maximal for the model
            top = int(logits[t][w].float().argmax())
            assert want[t, top] >= want[t].max() - 1.5e-2 * want[t].abs().max()


def test_decode_step_partial_layers_and_worker_batching():
    """Workers do not interact: a worker's logits do not depend on which
    other workers share the step (rows gathered and scattered per worker),
    and layers=0 reduces to norm(embed) @ lm_head."""
    from tests._tiny_model import CFG as c, base_weights
    wts = base_weights()
    nb = 2
    ids = torch.tensor([3, 17, 600])
    mk = lambda W: ([torch.zeros(W * nb, c.block, c.kv_heads, c.head_dim, dtype=BF16) for _ in range(c.layers)],  # noqa
                    [torch.zeros(W * nb, c.block, c.kv_heads, c.head_dim, dtype=BF16) for _ in range(c.layers)])
    cs = ref.cos_sin_cache(ref.rope_inv_freq(c.head_dim, c.theta), 64)
    kc, vc = mk(3)
    bt = torch.arange(3 * nb, dtype=torch.int32).reshape(3, nb)
    hn3, lg3 = ref.decode_step(c, wts, [None] * 3, kc, vc, bt, torch.zeros(3, dtype=torch.int32), ids, cs)
    kc1, vc1 = mk(1)
    hn1, lg1 = ref.decode_step(c, wts, [None], kc1, vc1, bt[:1], torch.zeros(1, dtype=torch.int32), ids[1:2], cs)
    assert rel_err(lg3[1], lg1[0]) <= 1e-2
    hn0, lg0 = ref.decode_step(c, wts, [None] * 3, kc, vc, bt, torch.zeros(3, dtype=torch.int32), ids, cs, layers=0)
    want = ref.rms_norm(wts["embed"][ids], wts["final_norm"], c.eps)
    assert bits_equal(hn0, want)
    assert bits_equal(lg0, ref.base_gemm(want, wts["lm_head"]))


def test_rope_inv_freq_llama3_scaling_matches_transformers():
    """Llama 3.1's rope_scaling (type llama3): the oracle's remap equals
    transformers' own initializer for that type, which is what the
    reference's LlamaRotaryEmbedding(config) calls (model_builder.py:293-296);
    the unscaled band and the factor-divided band are also checked by hand."""
    from transformers import LlamaConfig
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    sc = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}
    cfg = LlamaConfig(hidden_size=4096, num_attention_heads=32, head_dim=128, rope_theta=500000.0,
                      max_position_embeddings=131072, rope_scaling=dict(sc))
    want, _ = ROPE_INIT_FUNCTIONS["llama3"](cfg, "cpu")
    got = ref.rope_inv_freq(128, 500000.0, sc)
    assert torch.allclose(got, want.float(), rtol=1e-6, atol=0)
    plain = ref.rope_inv_freq(128, 500000.0)
    wl = 2 * math.pi / plain
    hi_band, lo_band = wl < 8192 / 4.0, wl > 8192 / 1.0
    assert hi_band.any() and lo_band.any() and (~hi_band & ~lo_band).any()
    assert torch.equal(got[hi_band], plain[hi_band])
    assert torch.allclose(got[lo_band], plain[lo_band] / 8.0, rtol=1e-7)


def test_worker_rotary_inv_freq_llama3_matches_oracle():
    """The worker's RotaryInvFreq (host-side torch) with the same scaling."""
    from swarmlora_amd.worker.paged_attention import RotaryInvFreq
    sc = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}
    assert torch.allclose(RotaryInvFreq(128, 500000.0, rope_scaling=sc).inv_freq,
                          ref.rope_inv_freq(128, 500000.0, sc), rtol=1e-6, atol=0)
    assert torch.equal(RotaryInvFreq(128, 500000.0).inv_freq, ref.rope_inv_freq(128, 500000.0))
    with pytest.raises(ValueError):
        RotaryInvFreq(128, 500000.0, rope_scaling={"rope_type": "yarn", "factor": 4.0})
