"""GPU tests of the round fusions (swl_round_ex_bf16, include/swl.h): each
fused round against the same round unfused followed by the worker-side step
it replaces, and against the CPU oracle.

The fused forms compute the worker-side step from the round's own bf16
output, so they are checked tightly against the unfused GPU round: the
residual add bit-exactly, RoPE / SiLU*up to one bf16 rounding, the RMSNorm on
staging (its per-row scale from fp32 partial sums) to 1e-3.  Against the
oracle the usual REL_TOL applies.
"""

import pytest
import torch

from oracle import reference_path as ref
from tests._util import BF16, REL_TOL, SEED_A, SEED_W, SEED_X, assert_close, bits_equal, randn, rel_err

pytestmark = pytest.mark.gpu

H, KV, HQ, HD, I = 4096, 8, 32, 128, 14336
QKV = (HQ + 2 * KV) * HD
T = 28
EPS = 1e-5


def _ops():
    from swarmlora_amd import ops
    return ops


def _table(dev, in_dim, out_dims, n, r=16, scale=2.0):
    ops = _ops()
    table = ops.LoraTable(dev)
    ads = []
    for i in range(n):
        blocks = [(randn((r, in_dim), SEED_A * 1000 + 10 * i + 2 * j, std=0.02),
                   randn((od, r), SEED_A * 1000 + 10 * i + 2 * j + 1, std=0.02)) for j, od in enumerate(out_dims)]
        table.add(torch.cat([A for A, _ in blocks], 0).contiguous().to(dev), [B.contiguous().to(dev) for _, B in blocks],
                  r, scale)
        ads.append([(A, B, scale) for A, B in blocks])
    return table, ads


def _ss_partials(rows: torch.Tensor, chunk=256) -> torch.Tensor:
    """fp32 sums of squares of each row over consecutive 256-column chunks."""
    f = rows.float()
    n = f.shape[1]
    return torch.stack([f[:, j:j + chunk].pow(2).sum(1) for j in range(0, n, chunk)], 1)


def _plain(dev, xs, w, out_dims, table, ads_ids):
    ops = _ops()
    n = w.shape[0]
    out = [torch.zeros(1, n, dtype=BF16, device=dev) for _ in xs]
    ops.round_fused([x.to(dev) for x in xs], out, [1] * len(xs), w.to(dev), None, seg_lora=ads_ids, table=table,
                    blk_cols=out_dims)
    return out


@pytest.mark.parametrize("in_dim,out_dims", [(H, [H, KV * HD, KV * HD]), (H, [I, I])])
def test_norm_on_staging(dev, in_dim, out_dims):
    """norm_weight: the round multiplies LlamaRMSNorm(h) built from ss_in."""
    ops = _ops()
    n = sum(out_dims)
    w = randn((n, in_dim), SEED_W, std=0.02)
    hs = [randn((1, in_dim), SEED_X * 100 + i, std=3.0) for i in range(T)]
    gamma = (1 + randn((in_dim,), 77, std=0.1).float()).to(BF16)
    table, ads = _table(dev, in_dim, out_dims, T)
    ids = list(range(T))
    hcat = torch.cat(hs, 0)
    ss = _ss_partials(hcat).to(dev)
    fz = ops.round_fusion(norm_weight=gamma.to(dev), eps=EPS, ss_in=ss)
    got = [torch.zeros(1, n, dtype=BF16, device=dev) for _ in range(T)]
    ops.round_ex([h.to(dev) for h in hs], got, [1] * T, w.to(dev), None, seg_lora=ids, table=table,
                 blk_cols=out_dims, fusion=fz)
    xn = [ref.rms_norm(h, gamma, EPS) for h in hs]
    unfused = _plain(dev, xn, w, out_dims, table, ids)
    torch.cuda.synchronize()
    op = ref.OP_QKV_FUSED if len(out_dims) == 3 else ref.OP_GATE_UP_FUSED
    want = ref.round_with_lora(op, xn, [1] * T, w, [ads[i] for i in ids], out_dims)
    for i in range(T):
        assert rel_err(got[i], unfused[i]) <= 1e-3, f"row {i}: fused vs unfused"
        assert_close(got[i], want[i], what=f"row {i} vs oracle")


@pytest.mark.parametrize("in_dim", [H, I])
def test_residual_and_sums_of_squares(dev, in_dim):
    """out_mode 1: h = bf16(h + out) bit-exactly as the unfused add, and the
    per-256-column sums of squares of the new h."""
    ops = _ops()
    w = randn((H, in_dim), SEED_W + 1, std=0.02)
    xs = [randn((1, in_dim), SEED_X * 200 + i) for i in range(T)]
    h0 = [randn((1, H), SEED_X * 300 + i, std=2.0) for i in range(T)]
    table, ads = _table(dev, in_dim, [H], T)
    ids = list(range(T))
    nss = H // 256
    ss = torch.full((T, nss + 3), -1.0, dtype=torch.float32, device=dev)
    fz = ops.round_fusion(out_mode=1, ss_out=ss)
    hd = [h.clone().to(dev) for h in h0]
    ops.round_ex([x.to(dev) for x in xs], hd, [1] * T, w.to(dev), None, seg_lora=ids, table=table, blk_cols=[H],
                 fusion=fz)
    unfused = _plain(dev, xs, w, [H], table, ids)
    torch.cuda.synchronize()
    want_base = ref.round_with_lora(ref.OP_O_PROJ, xs, [1] * T, w, [ads[i] for i in ids], [H])
    for i in range(T):
        hn = (h0[i].float() + unfused[i].cpu().float()).to(BF16)
        assert bits_equal(hd[i], hn), f"row {i}: residual add"
        assert_close(hd[i], (h0[i].float() + want_base[i].float()).to(BF16), what=f"row {i} vs oracle")
    got_ss = ss.cpu()
    want_ss = _ss_partials(torch.cat([h.cpu() for h in hd], 0))
    assert torch.allclose(got_ss[:, :nss], want_ss, rtol=1e-5, atol=1e-5)
    assert (got_ss[:, nss:] == -1.0).all(), "ss_out written past ceil(n / 256)"


def test_silu_mul_epilogue(dev):
    """out_mode 2: bf16(bf16(silu(gate)) * up) of the Gate+Up round output."""
    ops = _ops()
    w = randn((2 * I, H), SEED_W + 2, std=0.02)
    xs = [randn((1, H), SEED_X * 400 + i) for i in range(T)]
    table, ads = _table(dev, H, [I, I], T)
    ids = list(range(T))
    got = [torch.zeros(1, I, dtype=BF16, device=dev) for _ in range(T)]
    ops.round_ex([x.to(dev) for x in xs], got, [1] * T, w.to(dev), None, seg_lora=ids, table=table,
                 blk_cols=[I, I], fusion=ops.round_fusion(out_mode=2))
    unfused = _plain(dev, xs, w, [I, I], table, ids)
    torch.cuda.synchronize()
    want = ref.round_with_lora(ref.OP_GATE_UP_FUSED, xs, [1] * T, w, [ads[i] for i in ids], [I, I])
    for i in range(T):
        u = unfused[i].cpu()
        step = ref.silu_mul(u[:, :I], u[:, I:])
        d = (got[i].cpu().float() - step.float()).abs()
        assert (d <= step.float().abs() / 128 + 1e-30).all(), f"row {i}: more than one bf16 rounding off"
        # the gate / up halves the fused epilogue started from, against the
        # oracle (silu(g)*u of two outputs each within 1e-2 compounds both
        # errors, so the product itself is pinned by the step above)
        assert_close(u, want[i], what=f"row {i} gate|up vs oracle")


def test_rope_and_kv_append_epilogue(dev):
    """out_mode 3: rotated q / k in the row, k and v appended to the pages."""
    ops = _ops()
    w = randn((QKV, H), SEED_W + 3, std=0.02)
    xs = [randn((1, H), SEED_X * 500 + i) for i in range(T)]
    table, ads = _table(dev, H, [HQ * HD, KV * HD, KV * HD], T)
    ids = list(range(T))
    bs, mb = 16, 8
    nb = T * mb
    kc = randn((nb, bs, KV, HD), 900).to(dev)
    vc = randn((nb, bs, KV, HD), 901).to(dev)
    k0, v0 = kc.clone(), vc.clone()
    g = torch.Generator().manual_seed(5)
    bt = torch.randperm(nb, generator=g).to(torch.int32).reshape(T, mb)
    seql = torch.randint(0, mb * bs, (T,), generator=g).to(torch.int32)
    pos = seql.long() + torch.randint(0, 3, (T,), generator=g)
    pos[3] = -1                       # no rotation at an out-of-range position
    cs = ref.cos_sin_cache(ref.rope_inv_freq(HD, 500000.0), mb * bs + 4)
    fz = ops.round_fusion(out_mode=3, k_cache=kc, v_cache=vc, hq=HQ, hkv=KV, block_table=bt.to(dev),
                          cache_seqlens=seql.to(dev), positions=pos.to(dev), cos_sin=cs.to(dev))
    got = [torch.zeros(1, QKV, dtype=BF16, device=dev) for _ in range(T)]
    ops.round_ex([x.to(dev) for x in xs], got, [1] * T, w.to(dev), None, seg_lora=ids, table=table,
                 blk_cols=[HQ * HD, KV * HD, KV * HD], fusion=fz)
    unfused = _plain(dev, xs, w, [HQ * HD, KV * HD, KV * HD], table, ids)
    torch.cuda.synchronize()
    kc_c, vc_c = kc.cpu(), vc.cpu()
    k0c, v0c = k0.cpu(), v0.cpu()
    touched = set()
    for i in range(T):
        u = unfused[i].cpu().reshape(HQ + 2 * KV, HD)
        qk = u[:HQ + KV].unsqueeze(0)
        if pos[i] >= 0:
            qk = ref.rope_neox(qk, pos[i:i + 1], cs)
        want_row = torch.cat([qk[0], u[HQ + KV:]], 0).reshape(1, QKV)
        d = (got[i].cpu().float() - want_row.float()).abs()
        assert (d <= want_row.float().abs() / 128 + 1e-30).all(), f"row {i}: RoPE more than one rounding off"
        p = int(seql[i])
        blk = int(bt[i, p // bs])
        touched.add((blk, p % bs))
        assert bits_equal(kc_c[blk, p % bs], got[i].cpu().reshape(-1, HD)[HQ:HQ + KV]), f"row {i}: k page"
        assert bits_equal(vc_c[blk, p % bs], u[HQ + KV:]), f"row {i}: v page = unrotated v"
    # nothing else in the pages changed
    mask = torch.ones(nb, bs, dtype=torch.bool)
    for blk, off in touched:
        mask[blk, off] = False
    assert bits_equal(kc_c[mask], k0c[mask]) and bits_equal(vc_c[mask], v0c[mask])
    # and the oracle: q rotated from the reference round output
    want = ref.round_with_lora(ref.OP_QKV_FUSED, xs, [1] * T, w, [ads[i] for i in ids],
                               [HQ * HD, KV * HD, KV * HD])
    qw = torch.cat([wv.reshape(1, HQ + 2 * KV, HD)[:, :HQ] for wv in want], 0)
    qw = torch.where((pos >= 0).reshape(T, 1, 1), ref.rope_neox(qw, pos.clamp(min=0), cs), qw)
    qg = torch.cat([gv.cpu().reshape(1, HQ + 2 * KV, HD)[:, :HQ] for gv in got], 0)
    assert_close(qg, qw, what="rotated q vs oracle")


def test_fusion_rejects_bad_arguments(dev):
    ops = _ops()
    w = torch.zeros(H, H, dtype=BF16, device=dev)
    x = [torch.zeros(1, H, dtype=BF16, device=dev)]
    y = [torch.zeros(1, H, dtype=BF16, device=dev)]
    small = torch.zeros(1, 4, dtype=torch.float32, device=dev)   # needs 16 partials per row
    with pytest.raises(RuntimeError, match="ss_out"):
        ops.round_ex(x, y, [1], w, fusion=ops.round_fusion(out_mode=1, ss_out=small))
    xs = [torch.zeros(65, H, dtype=BF16, device=dev)]
    ys = [torch.zeros(65, H, dtype=BF16, device=dev)]
    ss = torch.zeros(65, 16, dtype=torch.float32, device=dev)
    with pytest.raises(RuntimeError, match="64 token rows"):
        ops.round_ex(xs, ys, [65], w, fusion=ops.round_fusion(out_mode=1, ss_out=ss))
