"""GPU parity of the libswl kernels against the CPU oracle.

Integer/byte work (gather, scatter, page append of v) must be bit-exact;
floating-point results must be within REL_TOL (normalised max error, see
tests/_util.py) of the oracle on the same seeded inputs.
"""

import math

import pytest
import torch

from oracle import reference_path as ref
from tests._util import (BF16, REL_TOL, SEED_A, SEED_META, SEED_W, SEED_X, assert_close, bits_equal, randn,
                         rel_err)

pytestmark = pytest.mark.gpu

H, KV, HD, I = 4096, 8, 128, 14336
QKV = H + 2 * KV * HD


def _ops():
    from swarmlora_amd import ops
    return ops


# ----------------------------------------------------------- gather/scatter --
@pytest.mark.parametrize("rows,d", [([1, 1, 1, 1], 4096), ([3, 0, 7, 1, 16], 4096), ([5, 2], 72), ([2, 3], 13)])
def test_gather_bit_exact(dev, rows, d):
    ops = _ops()
    slots = [randn((max(t, 1) + 2, d), SEED_X + i) for i, t in enumerate(rows)]
    packed = ops.gather([s.to(dev) for s in slots], rows)
    torch.cuda.synchronize()
    assert bits_equal(packed, ref.gather(slots, rows))


@pytest.mark.parametrize("rows,d", [([1, 1, 1, 1], 6144), ([4, 0, 9], 4096), ([3, 2], 20)])
def test_scatter_bit_exact_and_delta(dev, rows, d):
    ops = _ops()
    T = sum(rows)
    y = randn((T, d), SEED_X)
    delta = randn((T, d), SEED_A, std=0.1)
    outs = [torch.full((max(t, 1), d), -7.0, dtype=BF16, device=dev) for t in rows]
    ops.scatter_add(y.to(dev), outs, rows)
    torch.cuda.synchronize()
    expect = ref.scatter(y, rows)
    for o, e, t in zip(outs, expect, rows):
        assert bits_equal(o[:t], e)
        if t == 0:
            assert bool((o == -7.0).all())  # untouched
    ops.scatter_add(y.to(dev), outs, rows, delta=delta.to(dev))
    torch.cuda.synchronize()
    want = ref.scatter((y.float() + delta.float()).to(BF16), rows)  # one rounding of the fp32 sum
    for o, e, t in zip(outs, want, rows):
        assert bits_equal(o[:t], e)


# --------------------------------------------------------------------- GEMM --
@pytest.mark.parametrize("m", [1, 4, 16, 17, 28, 33, 64, 65, 200])
def test_gemm_matches_oracle(dev, m):
    ops = _ops()
    n, k = 768, 1024
    x = randn((m, k), SEED_X)
    w = randn((n, k), SEED_W, std=0.02)
    y = ops.gemm(x.to(dev), w.to(dev))
    torch.cuda.synchronize()
    assert_close(y, ref.base_gemm(x, w), what=f"gemm m={m}")
    # against an fp64 product too (the oracle itself rounds once to bf16)
    exact = (x.double() @ w.double().t())
    assert rel_err(y, exact) <= 5e-3


@pytest.mark.parametrize("m", [3, 100])
def test_gemm_bias_and_ragged_n(dev, m):
    ops = _ops()
    n, k = 200, 512   # n not a multiple of 16 / 128
    x = randn((m, k), SEED_X)
    w = randn((n, k), SEED_W, std=0.05)
    b = randn((n,), SEED_A)
    y = ops.gemm(x.to(dev), w.to(dev), b.to(dev))
    torch.cuda.synchronize()
    assert_close(y, ref.base_gemm(x, w, b), what="gemm+bias")


def test_gemm_one_hot_selects_weight_column_exactly(dev):
    """x = e_j picks W[:, j] exactly (no rounding anywhere)."""
    ops = _ops()
    n, k = 512, 4096
    w = randn((n, k), SEED_W)
    for m in (5, 80):
        idx = torch.arange(m) * 37 % k
        x = torch.zeros(m, k, dtype=BF16)
        x[torch.arange(m), idx] = 1.0
        y = ops.gemm(x.to(dev), w.to(dev))
        torch.cuda.synchronize()
        assert bits_equal(y, w[:, idx].t().contiguous())


@pytest.mark.parametrize("n,k", [(QKV, H), (H, H), (2 * I, H), (H, I)])
def test_gemm_full_decode_shapes(dev, n, k):
    """The four base projections at Llama-3.1-8B shape, 28 decode tokens."""
    ops = _ops()
    x = randn((28, k), SEED_X)
    w = randn((n, k), SEED_W, std=0.02)
    y = ops.gemm(x.to(dev), w.to(dev))
    torch.cuda.synchronize()
    assert_close(y, ref.base_gemm(x, w), what=f"gemm [{n}x{k}]")


# ------------------------------------------------------------------ rounds --
def _adapter(seed, r, in_dim, out_dims, std=0.02):
    """Per-block (A [r, in], B [out, r]) pairs ~N(0, std)."""
    blocks = []
    for j, od in enumerate(out_dims):
        A = randn((r, in_dim), seed * 100 + 2 * j, std=std)
        B = randn((od, r), seed * 100 + 2 * j + 1, std=std)
        blocks.append((A, B))
    return blocks


def _run_round(dev, rows, in_dim, out_dims, ranks, scale=2.0, adapter_ids=None, with_lora=True, bias=False):
    ops = _ops()
    n = sum(out_dims)
    w = randn((n, in_dim), SEED_W, std=0.02)
    b = randn((n,), SEED_W + 10) if bias else None
    xs = [randn((max(t, 1), in_dim), SEED_X * 1000 + i) for i, t in enumerate(rows)]
    n_adapters = (max(adapter_ids) + 1) if adapter_ids is not None else len(rows)
    adapters = [_adapter(SEED_A + 7 * i, ranks[i % len(ranks)], in_dim, out_dims) for i in range(n_adapters)]
    seg_ad = adapter_ids if adapter_ids is not None else list(range(len(rows)))

    table = ops.LoraTable(dev)
    for ad, r in zip(adapters, [ranks[i % len(ranks)] for i in range(n_adapters)]):
        a = torch.cat([A for A, _ in ad], 0).contiguous().to(dev)
        bs = [B.contiguous().to(dev) for _, B in ad]
        table.add(a, bs, r, scale)
    seg_in = [x.to(dev) for x in xs]
    seg_out = [torch.zeros(max(t, 1), n, dtype=BF16, device=dev) for t in rows]
    ops.round_fused(seg_in, seg_out, rows, w.to(dev), b.to(dev) if b is not None else None,
                    seg_lora=seg_ad if with_lora else None, table=table if with_lora else None,
                    blk_cols=out_dims if with_lora else None)
    torch.cuda.synchronize()

    if with_lora:
        op = ref.OP_QKV_FUSED if len(out_dims) > 1 else ref.OP_O_PROJ
        ad_ref = [[(A, B, scale) for A, B in adapters[seg_ad[i]]] for i in range(len(rows))]
        want = ref.round_with_lora(op, xs, rows, w, ad_ref, out_dims)
    else:
        want = ref.execute_round(xs, rows, w, b)
    if bias and with_lora:
        want = [wv + b for wv in want]
    for i, t in enumerate(rows):
        if t == 0:
            continue
        assert_close(seg_out[i][:t], want[i], what=f"round slot {i}")
    return seg_out, want


def test_round_config1_qkv_lora(dev):
    """fused QKV, 4 slots x 1 decode token, rank-16 LoRA on
    q/k/v per slot, scale 2.0."""
    _run_round(dev, [1, 1, 1, 1], H, [H, KV * HD, KV * HD], [16])


def test_round_no_lora_matches_execute_batched_gemm(dev):
    _run_round(dev, [1, 2, 1, 3], H, [H], [16], with_lora=False)


def test_round_single_slot_and_bias(dev):
    _run_round(dev, [1], H, [H], [16], with_lora=False, bias=True)
    _run_round(dev, [2], H, [H], [8], with_lora=True, bias=True)


@pytest.mark.parametrize("out_dims,in_dim", [([H], H), ([I, I], H), ([H], I)])
def test_round_decode_28_slots_each_projection(dev, out_dims, in_dim):
    """BASELINE config 2 rounds O, Gate+Up, Down at 28 slots x 1 token."""
    _run_round(dev, [1] * 28, in_dim, out_dims, [16])


def test_round_shared_adapters_zipf(dev):
    """BASELINE config 5 shape: 64 one-token slots drawing adapter ids from a
    Zipf(1.1) over a pool; slots sharing an adapter share its A/B."""
    g = torch.Generator().manual_seed(SEED_META)
    n_pool = 50
    p = torch.tensor([(i + 1) ** -1.1 for i in range(n_pool)])
    ids = torch.multinomial(p / p.sum(), 64, replacement=True, generator=g).tolist()
    used = sorted(set(ids))
    remap = {a: i for i, a in enumerate(used)}
    _run_round(dev, [1] * 64, H, [H, KV * HD, KV * HD], [16], adapter_ids=[remap[a] for a in ids])


@pytest.mark.parametrize("out_dims,in_dim", [([H, KV * HD, KV * HD], H), ([H], H), ([I, I], H), ([H], I)],
                         ids=["qkv", "o", "gate_up", "down"])
def test_round_config5_pool_of_500(dev, out_dims, in_dim):
    """BASELINE config 5 at full size, one round of the layer per case: 500
    rank-16 adapters ~N(0, 0.02) resident in HBM (drawn on the device from a
    seeded generator), 64 one-token slots drawing adapter ids from Zipf(1.1)
    over all 500; the table indexes the whole pool.  The oracle receives the
    adapters the slots use, copied back to the host."""
    ops = _ops()
    r, scale, n_pool, n_slots = 16, 2.0, 500, 64
    g = torch.Generator().manual_seed(SEED_META)
    p = torch.tensor([(i + 1) ** -1.1 for i in range(n_pool)])
    ids = torch.multinomial(p / p.sum(), n_slots, replacement=True, generator=g).tolist()
    gd = torch.Generator(device=dev).manual_seed(SEED_A)
    table = ops.LoraTable(dev)
    pool = []
    for _ in range(n_pool):
        a = (torch.randn(r * len(out_dims), in_dim, generator=gd, device=dev) * 0.02).to(BF16)
        bs = [(torch.randn(od, r, generator=gd, device=dev) * 0.02).to(BF16) for od in out_dims]
        table.add(a, bs, r, scale)
        pool.append((a, bs))
    n = sum(out_dims)
    w = randn((n, in_dim), SEED_W, std=0.02)
    xs = [randn((1, in_dim), SEED_X * 1000 + i) for i in range(n_slots)]
    seg_out = [torch.zeros(1, n, dtype=BF16, device=dev) for _ in range(n_slots)]
    ops.round_fused([x.to(dev) for x in xs], seg_out, [1] * n_slots, w.to(dev), None, seg_lora=ids, table=table,
                    blk_cols=out_dims)
    torch.cuda.synchronize()
    host = {}
    for a_id in set(ids):
        a, bs = pool[a_id]
        host[a_id] = [(a[j * r:(j + 1) * r].cpu(), b.cpu(), scale) for j, b in enumerate(bs)]
    op = ref.OP_QKV_FUSED if len(out_dims) > 1 else ref.OP_O_PROJ
    want = ref.round_with_lora(op, xs, [1] * n_slots, w, [host[a] for a in ids], out_dims)
    assert len(set(ids)) > 8 and max(ids) > 64  # shared adapters, ids beyond the slot count
    for i in range(n_slots):
        assert_close(seg_out[i], want[i], what=f"slot {i} (adapter {ids[i]})")


@pytest.mark.parametrize("ranks", [[8], [8, 16, 32, 64], [4, 12]])
def test_round_mixed_ranks_decode(dev, ranks):
    _run_round(dev, [1] * 9, H, [H, KV * HD, KV * HD], ranks)


def test_round_prefill_ragged_mixed_ranks(dev):
    """BASELINE config 3 (reduced): half the slots 1 token, the rest 32..160
    tokens, ranks from {8,16,32,64}; exercises the packed/tiled path."""
    g = torch.Generator().manual_seed(SEED_META)
    rows = [1, 1, 1, 1] + torch.randint(32, 161, (4,), generator=g).tolist()
    ranks = [[8, 16, 32, 64][int(i)] for i in torch.randint(0, 4, (8,), generator=g)]
    _run_round(dev, rows, H, [H, KV * HD, KV * HD], ranks)


@pytest.mark.parametrize("out_dims,in_dim", [([H, KV * HD, KV * HD], H), ([H], H), ([I, I], H), ([H], I)],
                         ids=["qkv", "o", "gate_up", "down"])
def test_round_config3_full_size(dev, out_dims, in_dim):
    """BASELINE config 3 at full size, one round of the layer per case: 16
    slots, half of them 1 token and the rest U{32..512} tokens (seeded),
    adapter ranks drawn from {8, 16, 32, 64}, scale 2.0.  Every row is checked
    against a float32 torch evaluation of the same per-slot products on the
    device; three rows of each slot (first, middle, last) against the oracle's
    bf16 restatement (rows are independent, so the oracle runs on those rows
    only)."""
    ops = _ops()
    g = torch.Generator().manual_seed(SEED_META + 3)
    rows = [1] * 8 + torch.randint(32, 513, (8,), generator=g).tolist()
    perm = torch.randperm(16, generator=g).tolist()
    rows = [rows[i] for i in perm]
    ranks = [[8, 16, 32, 64][int(i)] for i in torch.randint(0, 4, (16,), generator=g)]
    scale, n = 2.0, sum(out_dims)
    w = randn((n, in_dim), SEED_W, std=0.02)
    xs = [randn((t, in_dim), SEED_X * 1000 + i) for i, t in enumerate(rows)]
    ads = [_adapter(SEED_A + 7 * i, ranks[i], in_dim, out_dims) for i in range(16)]
    table = ops.LoraTable(dev)
    for ad, r in zip(ads, ranks):
        table.add(torch.cat([A for A, _ in ad], 0).contiguous().to(dev), [B.contiguous().to(dev) for _, B in ad], r,
                  scale)
    seg_out = [torch.zeros(t, n, dtype=BF16, device=dev) for t in rows]
    wd = w.to(dev)
    ops.round_fused([x.to(dev) for x in xs], seg_out, rows, wd, None, seg_lora=list(range(16)), table=table,
                    blk_cols=out_dims)
    torch.cuda.synchronize()
    wf = wd.float()
    for i, (x, ad) in enumerate(zip(xs, ads)):
        xf = x.to(dev).float()
        want = xf @ wf.t()
        c0 = 0
        for (A, B), od in zip(ad, out_dims):
            want[:, c0:c0 + od] += scale * ((xf @ A.to(dev).float().t()) @ B.to(dev).float().t())
            c0 += od
        assert_close(seg_out[i].float().cpu(), want.cpu(), what=f"slot {i} ({rows[i]} rows, rank {ranks[i]}) fp32")
    pick = [sorted({0, t // 2, t - 1}) for t in rows]
    op = ref.OP_QKV_FUSED if len(out_dims) > 1 else ref.OP_O_PROJ
    want = ref.round_with_lora(op, [x[p] for x, p in zip(xs, pick)], [len(p) for p in pick], w,
                               [[(A, B, scale) for A, B in ad] for ad in ads], out_dims)
    for i, p in enumerate(pick):
        assert_close(seg_out[i][p].cpu(), want[i], what=f"slot {i} rows {p} oracle")


def test_round_prefill_zero_row_segments(dev):
    _run_round(dev, [40, 0, 30, 0, 1], 1024, [512], [16])


# ----------------------------------------------------------- worker matmul --
@pytest.mark.parametrize("trans_b", [False, True])
def test_matmul_layouts(dev, trans_b):
    ops = _ops()
    m, k, n = 5, 4096, 48
    x = randn((m, k), SEED_X)
    b = randn((n, k) if trans_b else (k, n), SEED_W, std=0.02)
    y = ops.matmul(x.to(dev), b.to(dev), trans_b=trans_b, alpha=2.0)
    torch.cuda.synchronize()
    want = ((x @ (b.t() if trans_b else b)) * 2.0)
    assert_close(y, want, what="matmul")


@pytest.mark.parametrize("m,k,n,trans_b", [(1, 4096, 48, False), (1, 14336, 16, True), (1, 4096, 16, True),
                                             (7, 4096, 32, False), (64, 1024, 256, False), (3, 14336, 8, False),
                                             (2, 16384, 256, True), (1, 520, 40, True)])
def test_matmul_shrink_shapes(dev, m, k, n, trans_b):
    """The worker's LoRA shrink shapes (few columns, long rows: one
    workgroup per row, LDS-staged x) against a float32 evaluation of the
    same bf16 operands."""
    ops = _ops()
    x = randn((m, k), SEED_X)
    b = randn((n, k) if trans_b else (k, n), SEED_W, std=0.02)
    y = ops.matmul(x.to(dev), b.to(dev), trans_b=trans_b, alpha=2.0)
    torch.cuda.synchronize()
    want = (x.float() @ (b.float().t() if trans_b else b.float())) * 2.0
    assert_close(y, want, what=f"matmul {m}x{k}x{n} nt={trans_b}")


def test_matmul_shrink_unaligned_stride_takes_generic_path(dev):
    """A row stride that breaks 16-byte alignment is still computed (by the
    generic kernel) and agrees with the aligned case."""
    ops = _ops()
    m, k, n = 2, 4096, 16
    x = randn((m, k + 3), SEED_X)
    b = randn((n, k), SEED_W, std=0.02)
    xd = x.to(dev)
    y1 = ops.matmul(xd[:, :k], b.to(dev), trans_b=True)
    y2 = ops.matmul(xd[:, :k].contiguous(), b.to(dev), trans_b=True)
    torch.cuda.synchronize()
    want = x[:, :k].float() @ b.float().t()
    assert_close(y1, want, what="unaligned")
    assert_close(y2, want, what="aligned")


def test_matmul_strided_block_of_fused_B(dev):
    """A column block of a block-diagonal fused_B is read through its row stride."""
    ops = _ops()
    r, dims = 16, [64, 32, 32]
    fB = torch.zeros(3 * r, sum(dims), dtype=BF16)
    fB[r:2 * r, 64:96] = randn((r, 32), SEED_W)
    u = randn((4, 3 * r), SEED_X)
    fBd = fB.to(dev)
    y = ops.matmul(u.to(dev)[:, r:2 * r], fBd[r:2 * r, 64:96], trans_b=False)
    torch.cuda.synchronize()
    assert_close(y, u[:, r:2 * r] @ fB[r:2 * r, 64:96], what="strided block")


# ---------------------------------------------------------- paged attention --
def _attn_case(dev, nseq, L, ctx0, hq=32, hkv=8, bs=16, seed=0, shuffle=True):
    ops = _ops()
    d = 128
    max_pos = 4096
    g = torch.Generator().manual_seed(SEED_META + seed)
    max_blocks = (max(ctx0) + L + bs - 1) // bs + 1
    num_blocks = nseq * max_blocks + 3
    perm = torch.randperm(num_blocks, generator=g) if shuffle else torch.arange(num_blocks)
    bt = perm[: nseq * max_blocks].reshape(nseq, max_blocks).to(torch.int32)
    kc = randn((num_blocks, bs, hkv, d), 11 + seed)
    vc = randn((num_blocks, bs, hkv, d), 12 + seed)
    q = randn((nseq, L, hq, d), 13 + seed)
    k = randn((nseq, L, hkv, d), 14 + seed)
    v = randn((nseq, L, hkv, d), 15 + seed)
    seqlens = torch.tensor(ctx0, dtype=torch.int32)
    pos = (seqlens.long().unsqueeze(1) + torch.arange(L).unsqueeze(0)).reshape(-1)
    cs = ref.cos_sin_cache(ref.rope_inv_freq(d, 500000.0), max_pos)
    scale = 1.0 / math.sqrt(d)

    kc_d, vc_d, q_d, k_d, v_d = kc.to(dev), vc.to(dev), q.to(dev), k.to(dev), v.to(dev)
    out = ops.paged_attention(q_d, k_d, v_d, kc_d, vc_d, bt.to(dev), seqlens.to(dev), pos.to(dev), cs.to(dev),
                              scale)
    torch.cuda.synchronize()
    kc_r, vc_r = kc.clone(), vc.clone()
    want, q_rot, k_rot = ref.paged_attention(q, k, v, kc_r, vc_r, bt, seqlens, pos, cs, scale)
    return out, want, (q_d, k_d, kc_d, vc_d), (q_rot, k_rot, kc_r, vc_r)


@pytest.mark.parametrize("nseq,L,ctx0", [(3, 1, [0, 17, 100]), (2, 4, [5, 31]), (4, 1, [127, 128, 1000, 2047])])
def test_paged_attention_matches_oracle(dev, nseq, L, ctx0):
    out, want, got_state, ref_state = _attn_case(dev, nseq, L, ctx0)
    assert_close(out, want, what="attention out")
    q_d, k_d, kc_d, vc_d = got_state
    q_rot, k_rot, kc_r, vc_r = ref_state
    assert_close(q_d, q_rot, tol=1e-2, what="rope q in place")
    assert_close(k_d, k_rot, tol=1e-2, what="rope k in place")
    assert bits_equal(vc_d, vc_r), "v pages must be a bit-exact append"
    assert_close(kc_d, kc_r, what="k pages")


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (64, 8), (8, 2)])
def test_paged_attention_decode_gqa_groups(dev, hq, hkv):
    """One-token decode over contexts spanning many chunks (and a partial last
    chunk) for every supported q/kv head ratio."""
    out, want, got_state, ref_state = _attn_case(dev, 3, 1, [1, 300, 2047], hq=hq, hkv=hkv, seed=5)
    assert_close(out, want, what=f"attention hq={hq} hkv={hkv}")
    assert bits_equal(got_state[3], ref_state[3]), "v pages must be a bit-exact append"


@pytest.mark.parametrize("bs", [8, 32, 48])
def test_paged_attention_decode_block_sizes(dev, bs):
    """Pages of 8 keys (per-chunk kernel), 32 and 48 keys (16-key tiles
    inside a page, pages not a power of two) over contexts ending inside a
    tile, on a tile edge and past several parts."""
    out, want, got_state, ref_state = _attn_case(dev, 4, 1, [15, 16, 143, 1999], bs=bs, seed=9)
    assert_close(out, want, what=f"attention bs={bs}")
    assert bits_equal(got_state[3], ref_state[3]), "v pages must be a bit-exact append"


@pytest.mark.parametrize("nseq", [64, 70])
def test_paged_attention_decode_many_sequences(dev, nseq):
    """Decode over many ragged contexts: up to 64 sequences take the
    size-ordered part numbering (full parts first, then the partial last
    parts by length), more take the sequence-major one.  Contexts include
    0 keys, exactly one and two full 256-key parts (255 and 511 cached keys:
    the new key completes the part), one key past a part, and the rest drawn
    at random up to 700."""
    g = torch.Generator().manual_seed(77 + nseq)
    ctx0 = torch.randint(0, 701, (nseq,), generator=g).tolist()
    ctx0[:5] = [0, 255, 511, 256, 700]
    out, want, got_state, ref_state = _attn_case(dev, nseq, 1, ctx0, seed=21)
    assert_close(out, want, what=f"attention over {nseq} sequences")
    assert bits_equal(got_state[3], ref_state[3]), "v pages must be a bit-exact append"


def test_paged_attention_single_key_returns_v(dev):
    """ctx = 1: softmax over one key is 1, so the output is v exactly."""
    out, want, (q_d, k_d, kc_d, vc_d), _ = _attn_case(dev, 2, 1, [0, 0])
    v_new = randn((2, 1, 8, 128), 15)
    o = out.cpu().reshape(2, 32, 128)
    for h in range(32):
        assert bits_equal(o[:, h], v_new[:, 0, h // 4])


def test_paged_attention_page_permutation_invariant(dev):
    """Moving every physical page to another block id, together with the
    block table entries that name it, leaves the output unchanged."""
    ops = _ops()
    nseq, hq, hkv, d, bs = 2, 32, 8, 128, 16
    ctx0 = [200, 77]
    max_blocks = 14
    nb = nseq * max_blocks
    kc = randn((nb, bs, hkv, d), 21)
    vc = randn((nb, bs, hkv, d), 22)
    bt = torch.arange(nb).reshape(nseq, max_blocks).to(torch.int32)
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(7))
    kc_p, vc_p = torch.empty_like(kc), torch.empty_like(vc)
    kc_p[perm] = kc
    vc_p[perm] = vc
    bt_p = perm[bt.long()].to(torch.int32)
    q = randn((nseq, 1, hq, d), 23)
    k = randn((nseq, 1, hkv, d), 24)
    v = randn((nseq, 1, hkv, d), 25)
    sl = torch.tensor(ctx0, dtype=torch.int32)
    pos = sl.long()
    cs = ref.cos_sin_cache(ref.rope_inv_freq(d, 500000.0), 1024)
    outs = []
    for kcc, vcc, btt in ((kc, vc, bt), (kc_p, vc_p, bt_p)):
        outs.append(ops.paged_attention(q.to(dev), k.to(dev), v.to(dev), kcc.to(dev), vcc.to(dev), btt.to(dev),
                                        sl.to(dev), pos.to(dev), cs.to(dev), 1 / math.sqrt(d)))
    torch.cuda.synchronize()
    assert bits_equal(outs[0], outs[1])


def test_zero_blocks(dev):
    ops = _ops()
    caches = [randn((10, 16, 8, 128), s).to(dev) for s in range(4)]
    ids = torch.tensor([1, 7, 3], dtype=torch.int64, device=dev)
    ops.zero_blocks(caches, ids)
    torch.cuda.synchronize()
    for c in caches:
        assert float(c[[1, 7, 3]].abs().max()) == 0.0
        assert float(c[[0, 2, 4, 5, 6, 8, 9]].abs().min()) >= 0.0
        assert float(c[0].abs().max()) > 0.0


def test_captured_round_survives_scratch_growth(dev):
    """A decode-shaped round captured in a graph keeps reading valid scratch
    after later, larger prefill rounds grow the library's scratch area (the
    outgrown area stays allocated): every replay, with eager growth between
    replays, equals the eager result bit for bit."""
    ops = _ops()
    w = randn((H, H), SEED_W + 3, std=0.02).to(dev)
    xs = [randn((1, H), SEED_X + i).to(dev) for i in range(28)]
    want = [torch.zeros(1, H, dtype=BF16, device=dev) for _ in range(28)]
    ops.round_fused(xs, want, [1] * 28, w)
    got = [torch.zeros(1, H, dtype=BF16, device=dev) for _ in range(28)]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.round_fused(xs, got, [1] * 28, w)
    w2 = randn((512, H), SEED_W + 4, std=0.02).to(dev)
    gen = torch.Generator(device=dev).manual_seed(SEED_X + 50)
    for i in range(3):
        t = 4096 * (i + 2)  # each prefill round needs a larger packed staging area
        xb = torch.randn(t, H, generator=gen, device=dev, dtype=BF16)
        yb = torch.empty(t, 512, dtype=BF16, device=dev)
        ops.round_fused([xb], [yb], [t], w2)
        torch.cuda.synchronize()
        for o in got:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for j in range(28):
            assert bits_equal(got[j].cpu(), want[j].cpu()), f"replay {i} row {j}"
