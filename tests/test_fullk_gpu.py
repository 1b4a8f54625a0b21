"""GPU tests of the whole-K decode round (w_layout 2, fullk_kernel): one
launch per round, each workgroup holding the whole K range of the token rows
and finishing its tiles (LoRA shrink tiles first, then the weight tiles with
bias, LoRA expand and the out_mode fusion) without partial sums in memory.

Each case runs the same round through the K-sliced path (w_layout 1, split
and epilogue kernels, tested against the oracle elsewhere) and through the
whole-K path, on the same seeded inputs: the sums run in a different order,
so outputs agree to the bf16 rounding of their last step (normalised max
error well under 1e-2, measured ~4e-3 at most); each is also checked against
the CPU oracle at 1e-2.  Paired packing, repeated launches (the counters the
kernel resets), graph replays and the argument checks are covered too.
"""

import pytest
import torch

from oracle import reference_path as ref
from tests._util import BF16, REL_TOL, SEED_A, SEED_W, SEED_X, assert_close, bits_equal, randn, rel_err

pytestmark = pytest.mark.gpu

H, KV, HQ, HD, I = 4096, 8, 32, 128, 14336
QKV = (HQ + 2 * KV) * HD
EPS = 1e-5
AGREE = 5e-3  # whole-K vs K-sliced (one bf16 rounding apart)


def _ops():
    from swarmlora_amd import ops
    return ops


def _pack_cpu(w, off=8):
    """Fragment tiles with paired rows: tile t row r = W row paired(t, r)."""
    n, k = w.shape
    tiles = (n + 15) // 16
    per = off // 8
    rows = []
    for t in range(tiles):
        for r in range(16):
            rows.append((t // per) * 2 * off + (t % per) * 8 + (r & 7) + (off if r >= 8 else 0))
    wp = torch.zeros(tiles * 16, k, dtype=w.dtype)
    idx = torch.tensor(rows)
    ok = idx < n
    wp[ok.nonzero().flatten()] = w[idx[ok]]
    v = wp.view(tiles, 16, k // 32, 4, 8).permute(0, 2, 3, 1, 4)
    return v.contiguous().view(-1)


@pytest.mark.parametrize("n,k,off", [(256, 64, 64), (2 * 96, 96, 96), (4096, 4096, 8), (QKV, 1024, 64)])
def test_paired_pack_is_the_permuted_fragment_layout(dev, n, k, off):
    ops = _ops()
    w = randn((n, k), SEED_W + n + off, std=0.02)
    pw = ops.pack_weight(w.to(dev), pair_off=off)
    torch.cuda.synchronize()
    assert bits_equal(pw.data.cpu(), _pack_cpu(w, off))
    if off == 8:
        assert bits_equal(pw.data.cpu(), ops.pack_weight(w.to(dev)).data.cpu())


def _table(dev, in_dim, out_dims, n, ranks=None, scale=2.0, shared=None):
    """n adapters (rank ranks[i], default 16); shared: token -> adapter map."""
    ops = _ops()
    table = ops.LoraTable(dev)
    ads = []
    for i in range(n):
        r = ranks[i] if ranks else 16
        blocks = [(randn((r, in_dim), SEED_A * 1000 + 10 * i + 2 * j, std=0.02),
                   randn((od, r), SEED_A * 1000 + 10 * i + 2 * j + 1, std=0.02)) for j, od in enumerate(out_dims)]
        table.add(torch.cat([A for A, _ in blocks], 0).contiguous().to(dev), [B.contiguous().to(dev) for _, B in blocks],
                  r, scale)
        ads.append([(A, B, scale) for A, B in blocks])
    return table, ads


def _ss_partials(rows, chunk):
    f = rows.float()
    return torch.stack([f[:, j:j + chunk].pow(2).sum(1) for j in range(0, f.shape[1], chunk)], 1)


def _round(dev, layout, xs, ys, w_rows, out_dims, ids, table, **fz):
    """Run one round with weights in `layout` (1: K-sliced, 2: whole-K)."""
    ops = _ops()
    mode = fz.get("out_mode", 0)
    n = w_rows.shape[0]
    off = n // 2 if (layout == 2 and mode == 2) else 64 if (layout == 2 and mode == 3) else 8
    pw = ops.pack_weight(w_rows.to(dev), pair_off=off)
    f = ops.round_fusion(w_layout=layout, **fz)
    ops.round_ex(xs, ys, [1] * len(xs), pw, None, seg_lora=ids, table=table, blk_cols=out_dims if ids else None,
                 fusion=f)
    return pw


CASES = [
    # T, K, out_dims, lora ("distinct" | "shared" | None), norm
    (28, H, [HQ * HD, KV * HD, KV * HD], "distinct", False),
    (28, H, [H], "distinct", True),
    (1, H, [H], "distinct", False),
    (5, 1024, [512], None, True),
    (16, H, [2048], "shared", False),
    (17, 2048, [1024, 256, 256], "distinct", True),
    (32, H, [H], "mixed", True),
]


@pytest.mark.parametrize("T,K,out_dims,lora,norm", CASES)
def test_whole_k_mode0_matches_k_sliced_and_oracle(dev, T, K, out_dims, lora, norm):
    n = sum(out_dims)
    w = randn((n, K), SEED_W + T + K, std=0.02)
    hs = [randn((1, K), SEED_X * 100 + i, std=3.0 if norm else 1.0) for i in range(T)]
    ids, table, ads = None, None, None
    if lora == "distinct":
        table, ads = _table(dev, K, out_dims, T)
        ids = list(range(T))
    elif lora == "shared":
        table, ads = _table(dev, K, out_dims, 3)
        ids = [i % 3 for i in range(T)]
    elif lora == "mixed":
        table, ads = _table(dev, K, out_dims, 4, ranks=[8, 16, 32, 64])
        ids = [(i % 5) - 1 for i in range(T)]  # -1: no adapter
    fz = {}
    gamma = None
    if norm:
        gamma = (1 + randn((K,), 77, std=0.1).float()).to(BF16)
        fz = dict(norm_weight=gamma.to(dev), eps=EPS, ss_in=_ss_partials(torch.cat(hs, 0), 256).to(dev))
    xs = [h.to(dev) for h in hs]
    y1 = [torch.zeros(1, n, dtype=BF16, device=dev) for _ in range(T)]
    y2 = [torch.full((1, n), 7.0, dtype=BF16, device=dev) for _ in range(T)]
    _round(dev, 1, xs, y1, w, out_dims, ids, table, **fz)
    _round(dev, 2, xs, y2, w, out_dims, ids, table, **fz)
    torch.cuda.synchronize()
    g1 = torch.cat([y.cpu() for y in y1], 0)
    g2 = torch.cat([y.cpu() for y in y2], 0)
    e = rel_err(g2, g1)
    assert e <= AGREE, f"whole-K vs K-sliced: {e:.3e}"
    xn = [ref.rms_norm(h, gamma, EPS) for h in hs] if norm else hs
    op = ref.OP_QKV_FUSED if len(out_dims) == 3 else ref.OP_GATE_UP_FUSED if len(out_dims) == 2 else ref.OP_O_PROJ
    ad = [ads[i] if (ids and i >= 0) else None for i in (ids or [-1] * T)]
    want = ref.round_with_lora(op, xn, [1] * T, w, ad, out_dims)
    assert_close(g2, torch.cat(want, 0), what="whole-K vs oracle")


def test_whole_k_residual_and_sums_of_squares(dev):
    """out_mode 1: h = bf16(h + out) (one rounding of the K-sliced result at
    most) and n / 16 partial sums of squares of the new h per row."""
    ops = _ops()
    T = 28
    w = randn((H, H), SEED_W + 11, std=0.02)
    xs = [randn((1, H), SEED_X * 200 + i).to(dev) for i in range(T)]
    h0 = [randn((1, H), SEED_X * 300 + i, std=2.0) for i in range(T)]
    table, ads = _table(dev, H, [H], T)
    ids = list(range(T))
    ss1 = torch.zeros(T, H // 256, dtype=torch.float32, device=dev)
    ss2 = torch.full((T, H // 16 + 5), -1.0, dtype=torch.float32, device=dev)
    h1 = [h.clone().to(dev) for h in h0]
    h2 = [h.clone().to(dev) for h in h0]
    _round(dev, 1, xs, h1, w, [H], ids, table, out_mode=1, ss_out=ss1)
    _round(dev, 2, xs, h2, w, [H], ids, table, out_mode=1, ss_out=ss2)
    torch.cuda.synchronize()
    a, b = torch.cat([h.cpu() for h in h1], 0), torch.cat([h.cpu() for h in h2], 0)
    d = (a.float() - b.float()).abs()
    assert (d <= a.float().abs() / 64 + 1e-6).all(), "residual more than a rounding apart"
    got = ss2.cpu()
    assert torch.allclose(got[:, :H // 16], _ss_partials(b, 16), rtol=1e-5, atol=1e-5)
    assert (got[:, H // 16:] == -1.0).all(), "ss_out written past n / 16"
    want = ref.round_with_lora(ref.OP_O_PROJ, [x.cpu() for x in xs], [1] * T, w, [ads[i] for i in ids], [H])
    assert_close(b, torch.cat([(h0[i].float() + want[i].float()).to(BF16) for i in range(T)], 0),
                 what="residual vs oracle")


def test_whole_k_silu_mul(dev):
    """out_mode 2 over gate|up tiles packed with pair offset inter."""
    T = 28
    w = randn((2 * I, H), SEED_W + 12, std=0.02)
    xs = [randn((1, H), SEED_X * 400 + i).to(dev) for i in range(T)]
    table, ads = _table(dev, H, [I, I], T)
    ids = list(range(T))
    y1 = [torch.zeros(1, I, dtype=BF16, device=dev) for _ in range(T)]
    y2 = [torch.zeros(1, I, dtype=BF16, device=dev) for _ in range(T)]
    _round(dev, 1, xs, y1, w, [I, I], ids, table, out_mode=2)
    _round(dev, 2, xs, y2, w, [I, I], ids, table, out_mode=2)
    torch.cuda.synchronize()
    a, b = torch.cat([y.cpu() for y in y1], 0), torch.cat([y.cpu() for y in y2], 0)
    assert rel_err(b, a) <= AGREE
    want = ref.round_with_lora(ref.OP_GATE_UP_FUSED, [x.cpu() for x in xs], [1] * T, w, [ads[i] for i in ids],
                               [I, I])
    step = torch.cat([ref.silu_mul(u[:, :I], u[:, I:]) for u in want], 0)
    assert_close(b, step, tol=2 * REL_TOL, what="silu*up vs oracle (two compounded roundings)")


def test_whole_k_rope_and_kv_append(dev):
    """out_mode 3 over QKV tiles packed with pair offset 64: rotated q / k
    rows and the k / v pages as the K-sliced round writes them."""
    ops = _ops()
    T = 28
    w = randn((QKV, H), SEED_W + 13, std=0.02)
    xs = [randn((1, H), SEED_X * 500 + i).to(dev) for i in range(T)]
    table, ads = _table(dev, H, [HQ * HD, KV * HD, KV * HD], T)
    ids = list(range(T))
    bs, mb = 16, 8
    nb = T * mb
    g = torch.Generator().manual_seed(5)
    bt = torch.randperm(nb, generator=g).to(torch.int32).reshape(T, mb)
    seql = torch.randint(0, mb * bs, (T,), generator=g).to(torch.int32)
    pos = seql.long() + torch.randint(0, 3, (T,), generator=g)
    pos[3] = -1
    cs = ref.cos_sin_cache(ref.rope_inv_freq(HD, 500000.0), mb * bs + 4).to(dev)
    caches = []
    outs = []
    for layout in (1, 2):
        kc = randn((nb, bs, KV, HD), 900).to(dev)
        vc = randn((nb, bs, KV, HD), 901).to(dev)
        y = [torch.zeros(1, QKV, dtype=BF16, device=dev) for _ in range(T)]
        _round(dev, layout, xs, y, w, [HQ * HD, KV * HD, KV * HD], ids, table, out_mode=3, k_cache=kc, v_cache=vc,
               hq=HQ, hkv=KV, block_table=bt.to(dev), cache_seqlens=seql.to(dev), positions=pos.to(dev), cos_sin=cs)
        caches.append((kc, vc))
        outs.append(y)
    torch.cuda.synchronize()
    a = torch.cat([y.cpu() for y in outs[0]], 0)
    b = torch.cat([y.cpu() for y in outs[1]], 0)
    assert rel_err(b, a) <= AGREE
    (k1, v1), (k2, v2) = [(k.cpu(), v.cpu()) for k, v in caches]
    k0, v0 = randn((nb, bs, KV, HD), 900), randn((nb, bs, KV, HD), 901)
    mask = torch.ones(nb, bs, dtype=torch.bool)
    for i in range(T):
        p = int(seql[i])
        blk = int(bt[i, p // bs])
        mask[blk, p % bs] = False
        assert bits_equal(k2[blk, p % bs], b[i].reshape(-1, HD)[HQ:HQ + KV]), f"row {i}: k page = rotated k"
        assert bits_equal(v2[blk, p % bs], b[i].reshape(-1, HD)[HQ + KV:]), f"row {i}: v page = v"
        assert rel_err(k2[blk, p % bs], k1[blk, p % bs]) <= AGREE
    assert bits_equal(k2[mask], k0[mask]) and bits_equal(v2[mask], v0[mask]), "pages touched elsewhere"
    want = ref.round_with_lora(ref.OP_QKV_FUSED, [x.cpu() for x in xs], [1] * T, w, [ads[i] for i in ids],
                               [HQ * HD, KV * HD, KV * HD])
    qw = torch.cat([wv.reshape(1, HQ + 2 * KV, HD)[:, :HQ] for wv in want], 0)
    csc = cs.cpu()
    qw = torch.where((pos >= 0).reshape(T, 1, 1), ref.rope_neox(qw, pos.clamp(min=0), csc), qw)
    assert_close(b.reshape(T, HQ + 2 * KV, HD)[:, :HQ], qw, what="rotated q vs oracle")


@pytest.mark.parametrize("T", [28, 32])
def test_whole_k_norm_fused_lm_head(dev, T):
    """The LM head (vocab 128256, 8016 tiles over the persistent grid) with
    the final RMSNorm on the way in, against the K-sliced round."""
    V = 128256
    w = randn((V, H), SEED_W + 14, std=0.02)
    hs = [randn((1, H), SEED_X * 600 + i, std=2.0) for i in range(T)]
    gamma = (1 + randn((H,), 78, std=0.1).float()).to(BF16)
    ss = _ss_partials(torch.cat(hs, 0), 256).to(dev)
    xs = [h.to(dev) for h in hs]
    y1 = [torch.zeros(1, V, dtype=BF16, device=dev) for _ in range(T)]
    y2 = [torch.zeros(1, V, dtype=BF16, device=dev) for _ in range(T)]
    _round(dev, 1, xs, y1, w, [V], None, None, norm_weight=gamma.to(dev), eps=EPS, ss_in=ss)
    _round(dev, 2, xs, y2, w, [V], None, None, norm_weight=gamma.to(dev), eps=EPS, ss_in=ss)
    torch.cuda.synchronize()
    a, b = torch.cat([y.cpu() for y in y1], 0), torch.cat([y.cpu() for y in y2], 0)
    assert rel_err(b, a) <= AGREE
    xn = torch.cat([ref.rms_norm(h, gamma, EPS) for h in hs[:3]], 0)
    assert_close(b[:3], (xn.float() @ w.float().t()), what="LM head rows vs float32")


def test_whole_k_repeated_launches_and_graph_replays(dev):
    """The shrink-tile counter is reset by every launch: three eager rounds
    and three graph replays (eager work and synchronisation between them)
    give the same bits."""
    ops = _ops()
    T = 28
    out_dims = [H]
    w = randn((H, H), SEED_W + 15, std=0.02)
    xs = [randn((1, H), SEED_X * 700 + i).to(dev) for i in range(T)]
    table, _ = _table(dev, H, out_dims, T)
    ids = list(range(T))
    pw = ops.pack_weight(w.to(dev))
    f = ops.round_fusion(w_layout=2)
    ys = [torch.zeros(1, H, dtype=BF16, device=dev) for _ in range(T)]
    runs = []
    for _ in range(3):
        for y in ys:
            y.zero_()
        ops.round_ex(xs, ys, [1] * T, pw, None, seg_lora=ids, table=table, blk_cols=out_dims, fusion=f)
        torch.cuda.synchronize()
        runs.append(torch.cat([y.cpu() for y in ys], 0))
    assert all(bits_equal(r, runs[0]) for r in runs[1:])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ops.round_ex(xs, ys, [1] * T, pw, None, seg_lora=ids, table=table, blk_cols=out_dims, fusion=f)
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        for y in ys:
            y.fill_(3.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert bits_equal(torch.cat([y.cpu() for y in ys], 0), runs[0])


def test_whole_k_rejects_unsupported_shapes(dev):
    ops = _ops()
    w = ops.pack_weight(torch.zeros(64, 4096, dtype=BF16, device=dev))
    f = ops.round_fusion(w_layout=2)
    x33 = [torch.zeros(1, 4096, dtype=BF16, device=dev) for _ in range(33)]
    y33 = [torch.zeros(1, 64, dtype=BF16, device=dev) for _ in range(33)]
    with pytest.raises(RuntimeError, match="at most 32 token rows"):
        ops.round_ex(x33, y33, [1] * 33, w, None, fusion=f)
    w2 = ops.pack_weight(torch.zeros(64, 8192, dtype=BF16, device=dev))
    x8k = [torch.zeros(1, 8192, dtype=BF16, device=dev)]
    with pytest.raises(RuntimeError, match="multiple of 256, at most 4096"):
        ops.round_ex(x8k, y33[:1], [1], w2, None, fusion=f)
    w3 = ops.pack_weight(torch.zeros(40, 4096, dtype=BF16, device=dev))
    with pytest.raises(RuntimeError, match="multiple of 16"):
        ops.round_ex(x33[:1], y33[:1], [1], w3, None, fusion=f)
