"""GPU tests of the persistent decode chain (swl_chain_*, ops.ChainPlan): one
launch that runs dependent decode rounds as phases of a persistent grid.

Each round kind (residual with per-16-column sums of squares, RMSNorm on the
way in with SiLU * up, residual over k = 14336 with the token rows streamed,
RoPE with the KV-page append) runs as a one-round chain and through the
K-sliced round (w_layout 1, split and epilogue kernels, itself tested
against the oracle) on the same seeded inputs, at Llama-3.1-8B widths with
28 tokens and a distinct rank-16 adapter each: the sums run in a different
order, so the two agree to the bf16 rounding of their last step (normalised
max error <= 5e-3); each is also checked against the CPU oracle at 1e-2.
The whole-layer sequence (O, Gate+Up, Down, next QKV) runs in the config-4
decode test (tests/test_decode_config4_gpu.py, chain=True) against the
oracle's decode step.  Repeated launches and graph replays give the same
bits, the status word reports no expired wait, and unsupported shapes are
refused before launch.
"""

import pytest
import torch

from oracle import reference_path as ref
from tests._util import BF16, REL_TOL, SEED_A, SEED_W, SEED_X, assert_close, bits_equal, randn, rel_err

pytestmark = pytest.mark.gpu

H, KV, HQ, HD, I = 4096, 8, 32, 128, 14336
QKV = (HQ + 2 * KV) * HD
EPS = 1e-5
AGREE = 5e-3
T = 28


def _ops():
    from swarmlora_amd import ops
    return ops


def _table(dev, in_dim, out_dims, n, table=None, seed=0):
    """n rank-16 adapters (added to `table`, or a new one); their entry
    indices are len(table) before the call + 0..n-1."""
    ops = _ops()
    table = table if table is not None else ops.LoraTable(dev)
    ads = []
    for i in range(n):
        blocks = [(randn((16, in_dim), SEED_A * 1000 + seed + 10 * i + 2 * j, std=0.02),
                   randn((od, 16), SEED_A * 1000 + seed + 10 * i + 2 * j + 1, std=0.02))
                  for j, od in enumerate(out_dims)]
        table.add(torch.cat([A for A, _ in blocks], 0).contiguous().to(dev), [B.contiguous().to(dev) for _, B in blocks],
                  16, 2.0)
        ads.append([(A, B, 2.0) for A, B in blocks])
    return table, ads


def _ss16(rows):
    f = rows.float()
    return torch.stack([f[:, j:j + 16].pow(2).sum(1) for j in range(0, f.shape[1], 16)], 1)


def _ss256(rows):
    f = rows.float()
    return torch.stack([f[:, j:j + 256].pow(2).sum(1) for j in range(0, f.shape[1], 256)], 1)


def _run_chain(dev, rounds, table, kv=None):
    ops = _ops()
    plan = ops.ChainPlan(T, rounds, table=table, kv=kv)
    try:
        plan.launch()
        assert plan.status() == 0, "a device-side wait of the chain ran out"
    finally:
        plan.close()


@pytest.mark.parametrize("k", [H, I])
def test_chain_residual_round(dev, k):
    """out_mode 1: y = bf16(res + out) and one sum of squares per 16 columns;
    k = 14336 streams the token rows (the Down round)."""
    ops = _ops()
    w = randn((H, k), SEED_W + k, std=0.02)
    xs = randn((T, k), SEED_X * 10 + 1)
    res = randn((T, H), SEED_X * 10 + 2, std=2.0)
    table, ads = _table(dev, k, [H], T)
    ids = list(range(T))
    x_d, res_d = xs.to(dev), res.to(dev)
    y = torch.full((T, H), 5.0, dtype=BF16, device=dev)
    ss = torch.full((T, H // 16 + 3), -1.0, dtype=torch.float32, device=dev)
    print(f"chain residual round k={k}", flush=True)
    _run_chain(dev, [dict(w=ops.pack_weight(w.to(dev)), out_mode=1, x=x_d, y=y, res=res_d, ss_out=ss, lora=ids,
                          blk_cols=[H])], table)
    # K-sliced round: h += out in place
    h = res_d.clone()
    ss1 = torch.zeros(T, H // 256, dtype=torch.float32, device=dev)
    ops.round_ex([x_d[i:i + 1] for i in range(T)], [h[i:i + 1] for i in range(T)], [1] * T,
                 ops.pack_weight(w.to(dev)), None, seg_lora=ids, table=table, blk_cols=[H],
                 fusion=ops.round_fusion(out_mode=1, ss_out=ss1))
    torch.cuda.synchronize()
    got, ks = y.cpu(), h.cpu()
    # y = res + out is compared as out: near-cancelling elements make an
    # elementwise relative bound meaningless at k = 14336 (|out| ~ 2.4)
    e = rel_err(got.float() - res.float(), ks.float() - res.float())
    print(f"  chain vs K-sliced (out part): {e:.2e}", flush=True)
    assert e <= AGREE, f"chain vs K-sliced: {e:.3e}"
    gss = ss.cpu()
    assert torch.allclose(gss[:, :H // 16], _ss16(got), rtol=1e-5, atol=1e-5)
    assert (gss[:, H // 16:] == -1.0).all(), "ss_out written past n / 16"
    want = ref.round_with_lora(ref.OP_O_PROJ, [xs[i:i + 1] for i in range(T)], [1] * T, w, [ads[i] for i in ids], [H])
    assert_close(got, torch.cat([(res[i:i + 1].float() + want[i].float()).to(BF16) for i in range(T)], 0),
                 what="residual vs oracle")


def test_chain_norm_silu_round(dev):
    """out_mode 2 with RMSNorm on the way in (factors from 256 partial sums
    of squares per row): SiLU(gate) * up."""
    ops = _ops()
    w = randn((2 * I, H), SEED_W + 21, std=0.02)
    hs = randn((T, H), SEED_X * 20 + 1, std=2.0)
    gamma = (1 + randn((H,), 79, std=0.1).float()).to(BF16)
    table, ads = _table(dev, H, [I, I], T)
    ids = list(range(T))
    h_d = hs.to(dev)
    y = torch.zeros(T, I, dtype=BF16, device=dev)
    print("chain norm + silu round", flush=True)
    _run_chain(dev, [dict(w=ops.pack_weight(w.to(dev), pair_off=I), out_mode=2, x=h_d, y=y,
                          norm_weight=gamma.to(dev), ss_in=_ss16(hs).to(dev), eps=EPS, lora=ids,
                          blk_cols=[I, I])], table)
    y1 = torch.zeros(T, I, dtype=BF16, device=dev)
    ops.round_ex([h_d[i:i + 1] for i in range(T)], [y1[i:i + 1] for i in range(T)], [1] * T,
                 ops.pack_weight(w.to(dev)), None, seg_lora=ids, table=table, blk_cols=[I, I],
                 fusion=ops.round_fusion(norm_weight=gamma.to(dev), eps=EPS, ss_in=_ss256(hs).to(dev), out_mode=2))
    torch.cuda.synchronize()
    got = y.cpu()
    assert rel_err(got, y1.cpu()) <= AGREE
    xn = [ref.rms_norm(hs[i:i + 1], gamma, EPS) for i in range(T)]
    want = ref.round_with_lora(ref.OP_GATE_UP_FUSED, xn, [1] * T, w, [ads[i] for i in ids], [I, I])
    step = torch.cat([ref.silu_mul(u[:, :I], u[:, I:]) for u in want], 0)
    assert_close(got, step, tol=2 * REL_TOL, what="silu*up vs oracle (two compounded roundings)")


def test_chain_rope_round(dev):
    """out_mode 3: rotated q / k rows and the k / v pages as the K-sliced
    round writes them (RMSNorm on the way in)."""
    ops = _ops()
    w = randn((QKV, H), SEED_W + 22, std=0.02)
    hs = randn((T, H), SEED_X * 30 + 1, std=2.0)
    gamma = (1 + randn((H,), 80, std=0.1).float()).to(BF16)
    table, ads = _table(dev, H, [HQ * HD, KV * HD, KV * HD], T)
    ids = list(range(T))
    bs, mb = 16, 8
    nb = T * mb
    g = torch.Generator().manual_seed(6)
    bt = torch.randperm(nb, generator=g).to(torch.int32).reshape(T, mb)
    seql = torch.randint(0, mb * bs, (T,), generator=g).to(torch.int32)
    pos = seql.long() + torch.randint(0, 3, (T,), generator=g)
    pos[4] = -1
    cs = ref.cos_sin_cache(ref.rope_inv_freq(HD, 500000.0), mb * bs + 4).to(dev)
    h_d = hs.to(dev)
    outs, caches = [], []
    for layout in ("chain", "sliced"):
        kc = randn((nb, bs, KV, HD), 910).to(dev)
        vc = randn((nb, bs, KV, HD), 911).to(dev)
        kv = dict(k_cache=kc, v_cache=vc, hq=HQ, hkv=KV, block_table=bt.to(dev), cache_seqlens=seql.to(dev),
                  positions=pos.to(dev), cos_sin=cs)
        y = torch.zeros(T, QKV, dtype=BF16, device=dev)
        if layout == "chain":
            print("chain rope round", flush=True)
            _run_chain(dev, [dict(w=ops.pack_weight(w.to(dev), pair_off=64), out_mode=3, x=h_d, y=y,
                                  norm_weight=gamma.to(dev), ss_in=_ss16(hs).to(dev), eps=EPS, lora=ids,
                                  blk_cols=[HQ * HD, KV * HD, KV * HD])], table,
                       kv=ops.round_fusion(out_mode=3, **kv))
        else:
            ops.round_ex([h_d[i:i + 1] for i in range(T)], [y[i:i + 1] for i in range(T)], [1] * T,
                         ops.pack_weight(w.to(dev)), None, seg_lora=ids, table=table,
                         blk_cols=[HQ * HD, KV * HD, KV * HD],
                         fusion=ops.round_fusion(norm_weight=gamma.to(dev), eps=EPS, ss_in=_ss256(hs).to(dev),
                                                 out_mode=3, **kv))
        outs.append(y)
        caches.append((kc, vc))
    torch.cuda.synchronize()
    a, b = outs[0].cpu(), outs[1].cpu()
    assert rel_err(a, b) <= AGREE
    (k1, v1), (k2, v2) = [(k.cpu(), v.cpu()) for k, v in caches]
    k0, v0 = randn((nb, bs, KV, HD), 910), randn((nb, bs, KV, HD), 911)
    mask = torch.ones(nb, bs, dtype=torch.bool)
    for i in range(T):
        p = int(seql[i])
        blk = int(bt[i, p // bs])
        mask[blk, p % bs] = False
        assert bits_equal(k1[blk, p % bs], a[i].reshape(-1, HD)[HQ:HQ + KV]), f"row {i}: k page = rotated k"
        assert bits_equal(v1[blk, p % bs], a[i].reshape(-1, HD)[HQ + KV:]), f"row {i}: v page = v"
    assert bits_equal(k1[mask], k0[mask]) and bits_equal(v1[mask], v0[mask]), "pages touched elsewhere"
    xn = [ref.rms_norm(hs[i:i + 1], gamma, EPS) for i in range(T)]
    want = ref.round_with_lora(ref.OP_QKV_FUSED, xn, [1] * T, w, [ads[i] for i in ids], [HQ * HD, KV * HD, KV * HD])
    qw = torch.cat([wv.reshape(1, HQ + 2 * KV, HD)[:, :HQ] for wv in want], 0)
    qw = torch.where((pos >= 0).reshape(T, 1, 1), ref.rope_neox(qw, pos.clamp(min=0), cs.cpu()), qw)
    assert_close(a.reshape(T, HQ + 2 * KV, HD)[:, :HQ], qw, what="rotated q vs oracle")


def test_chain_layer_sequence_repeats_and_replays(dev):
    """The decode layer's four-round sequence at Llama-3.1-8B widths (Down
    streams its 14336-wide rows): three eager launches and three graph
    replays give identical bits, the status word stays 0, and the outputs
    equal the rounds run one by one as K-sliced rounds within the
    two-evaluation tolerance."""
    ops = _ops()
    h, inter, hq, hkv = H, I, HQ, KV
    qkv = (hq + 2 * hkv) * HD
    gd = torch.Generator(device=dev).manual_seed(31)
    rd = lambda *sh, std=0.02: (torch.randn(*sh, generator=gd, device=dev) * std).to(BF16)  # noqa: E731
    wo, wgu, wd, wq = rd(h, h), rd(2 * inter, h), rd(h, inter), rd(qkv, h)
    g1 = (1 + rd(h, std=0.1).float()).to(BF16)
    g2 = (1 + rd(h, std=0.1).float()).to(BF16)
    attn = rd(T, h, std=1.0)
    h0 = rd(T, h, std=2.0)
    # one table holding every round's entries
    table = ops.LoraTable(dev)
    base = {}
    for nm, k, dims, sd in (("o", h, [h], 0), ("gu", h, [inter, inter], 300), ("d", inter, [h], 600),
                            ("q", h, [hq * HD, hkv * HD, hkv * HD], 900)):
        base[nm] = len(table)
        _table(dev, k, dims, T, table=table, seed=sd)
    ids = lambda nm: [base[nm] + i for i in range(T)]  # noqa: E731
    bs, mb = 16, 4
    nb = T * mb
    bt = torch.arange(nb, dtype=torch.int32).reshape(T, mb).to(dev)
    seql = torch.full((T,), 20, dtype=torch.int32, device=dev)
    pos = seql.long()
    cs = ref.cos_sin_cache(ref.rope_inv_freq(HD, 500000.0), mb * bs).to(dev)
    kc = torch.zeros(nb, bs, hkv, HD, dtype=BF16, device=dev)
    vc = torch.zeros_like(kc)
    hm = torch.zeros(T, h, dtype=BF16, device=dev)
    hout = torch.zeros_like(hm)
    act = torch.zeros(T, inter, dtype=BF16, device=dev)
    y = torch.zeros(T, qkv, dtype=BF16, device=dev)
    ss_o = torch.zeros(T, h // 16, dtype=torch.float32, device=dev)
    ss_d = torch.zeros_like(ss_o)
    rounds = [dict(w=ops.pack_weight(wo), out_mode=1, x=attn, y=hm, res=h0, ss_out=ss_o, lora=ids("o"),
                   blk_cols=[h]),
              dict(w=ops.pack_weight(wgu, pair_off=inter), out_mode=2, x=hm, y=act, norm_weight=g1,
                   ss_in=ss_o, eps=EPS, lora=ids("gu"), blk_cols=[inter, inter]),
              dict(w=ops.pack_weight(wd), out_mode=1, x=act, y=hout, res=hm, ss_out=ss_d, lora=ids("d"),
                   blk_cols=[h]),
              dict(w=ops.pack_weight(wq, pair_off=64), out_mode=3, x=hout, y=y, norm_weight=g2, ss_in=ss_d,
                   eps=EPS, lora=ids("q"), blk_cols=[hq * HD, hkv * HD, hkv * HD])]
    kvf = ops.round_fusion(out_mode=3, k_cache=kc, v_cache=vc, hq=hq, hkv=hkv, block_table=bt, cache_seqlens=seql,
                           positions=pos, cos_sin=cs)
    plan = ops.ChainPlan(T, rounds, table=table, kv=kvf)
    try:
        runs = []
        for r in range(3):
            print(f"chain layer sequence: eager launch {r}", flush=True)
            for t in (hm, hout, act, y):
                t.fill_(7.0)
            plan.launch()
            torch.cuda.synchronize()
            runs.append([t.cpu() for t in (hm, act, hout, y)])
        assert plan.status() == 0
        for r in runs[1:]:
            assert all(bits_equal(a, b) for a, b in zip(r, runs[0])), "eager launches differ"
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(gr, stream=s):
                plan.launch()
        torch.cuda.current_stream().wait_stream(s)
        for r in range(3):
            print(f"chain layer sequence: graph replay {r}", flush=True)
            for t in (hm, hout, act, y):
                t.fill_(3.0)
            torch.cuda.synchronize()
            gr.replay()
            torch.cuda.synchronize()
            got = [t.cpu() for t in (hm, act, hout, y)]
            assert all(bits_equal(a, b) for a, b in zip(got, runs[0])), "graph replay differs"
        assert plan.status() == 0
        # the same four rounds one by one (K-sliced rounds)
        hh = h0.clone()
        s1 = torch.zeros(T, h // 256, dtype=torch.float32, device=dev)
        one = [1] * T
        rw = lambda t: [t[i:i + 1] for i in range(T)]  # noqa: E731
        ops.round_ex(rw(attn), rw(hh), one, ops.pack_weight(wo), None, seg_lora=ids("o"), table=table,
                     blk_cols=[h], fusion=ops.round_fusion(out_mode=1, ss_out=s1))
        a1 = torch.zeros(T, inter, dtype=BF16, device=dev)
        ops.round_ex(rw(hh), rw(a1), one, ops.pack_weight(wgu), None, seg_lora=ids("gu"), table=table,
                     blk_cols=[inter, inter], fusion=ops.round_fusion(norm_weight=g1, eps=EPS, ss_in=s1, out_mode=2))
        s2 = torch.zeros_like(s1)
        hh2 = hh.clone()
        ops.round_ex(rw(a1), rw(hh2), one, ops.pack_weight(wd), None, seg_lora=ids("d"), table=table,
                     blk_cols=[h], fusion=ops.round_fusion(out_mode=1, ss_out=s2))
        torch.cuda.synchronize()
        assert rel_err(runs[0][0], hh.cpu()) <= AGREE
        assert rel_err(runs[0][1], a1.cpu()) <= 2 * AGREE
        assert rel_err(runs[0][2], hh2.cpu()) <= 2 * AGREE
    finally:
        plan.close()


def test_chain_rejects_unsupported(dev):
    ops = _ops()
    w = ops.pack_weight(torch.zeros(64, 4096, dtype=BF16, device=dev))
    x = torch.zeros(33, 4096, dtype=BF16, device=dev)
    y = torch.zeros(33, 64, dtype=BF16, device=dev)
    with pytest.raises(RuntimeError, match="1..32 token rows"):
        ops.ChainPlan(33, [dict(w=w, out_mode=1, x=x, y=y, res=y)])
    w2 = ops.pack_weight(torch.zeros(64, 1024, dtype=BF16, device=dev))
    with pytest.raises(RuntimeError, match="supported round sequences"):
        ops.ChainPlan(4, [dict(w=w2, out_mode=1, x=x[:, :1024], y=y, res=y),
                          dict(w=w2, out_mode=1, x=x[:, :1024], y=y, res=y)])
    w3 = ops.pack_weight(torch.zeros(64, 8192, dtype=BF16, device=dev))
    x3 = torch.zeros(4, 8192, dtype=BF16, device=dev)
    ss = torch.zeros(4, 16, dtype=torch.float32, device=dev)
    with pytest.raises(RuntimeError, match="RMSNorm on the way in needs k <= 4096"):
        ops.ChainPlan(4, [dict(w=w3, out_mode=1, x=x3, y=y, res=y, norm_weight=torch.ones(8192, dtype=BF16,
                                                                                          device=dev), ss_in=ss)])
    w4 = ops.pack_weight(torch.zeros(64, 4096, dtype=BF16, device=dev))
    t = ops.LoraTable(dev)
    t.add(torch.zeros(8, 4096, dtype=BF16, device=dev), [torch.zeros(64, 8, dtype=BF16, device=dev)], 8, 1.0)
    with pytest.raises(RuntimeError, match="rank 16"):
        ops.ChainPlan(4, [dict(w=w4, out_mode=1, x=x[:4], y=y, res=y, lora=[0, 0, 0, 0], blk_cols=[64])], table=t)
