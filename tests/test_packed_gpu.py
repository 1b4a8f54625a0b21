"""GPU tests of the fragment-tile weight layout (swl_pack_weight_bf16,
swl_round_fusion.w_layout, include/swl.h).

The packing is a pure permutation, checked bit-exactly against the layout
restated with torch indexing on the CPU.  A round over the packed weight
multiplies the same numbers in the same order as the row-major round, so its
outputs are checked bit-identical to the row-major round's (shapes with N not
a multiple of 16, LoRA adapters, the norm-on-staging and residual fusions),
and against the oracle at the usual tolerance.
"""

import pytest
import torch

from oracle import reference_path as ref
from tests._util import BF16, SEED_W, SEED_X, assert_close, bits_equal, randn

pytestmark = pytest.mark.gpu


def _ops():
    from swarmlora_amd import ops
    return ops


def _pack_cpu(w: torch.Tensor) -> torch.Tensor:
    """Fragment tiles of w [n, k]: [tile][step][lane][8], lane l holding row
    16 * tile + l % 16 and columns 32 * step + 8 * (l // 16) .. + 7."""
    n, k = w.shape
    tiles = (n + 15) // 16
    wp = torch.zeros(tiles * 16, k, dtype=w.dtype)
    wp[:n] = w
    # [tile, r, step, q, e] -> [tile, step, q, r, e] (lane = q * 16 + r)
    v = wp.view(tiles, 16, k // 32, 4, 8).permute(0, 2, 3, 1, 4)
    return v.contiguous().view(-1)


@pytest.mark.parametrize("n,k", [(64, 64), (40, 96), (4096, 4096), (1000, 14336)])
def test_pack_is_the_fragment_permutation(dev, n, k):
    ops = _ops()
    w = randn((n, k), SEED_W + n, std=0.02)
    pw = ops.pack_weight(w.to(dev))
    torch.cuda.synchronize()
    assert pw.shape == (n, k)
    assert bits_equal(pw.data.cpu(), _pack_cpu(w))


def _table(dev, in_dim, out_dims, n, r=16, scale=2.0):
    ops = _ops()
    table = ops.LoraTable(dev)
    ads = []
    for i in range(n):
        blocks = [(randn((r, in_dim), 9000 + 10 * i + 2 * j, std=0.02),
                   randn((od, r), 9000 + 10 * i + 2 * j + 1, std=0.02)) for j, od in enumerate(out_dims)]
        table.add(torch.cat([A for A, _ in blocks], 0).contiguous().to(dev), [B.contiguous().to(dev) for _, B in blocks],
                  r, scale)
        ads.append([(A, B, scale) for A, B in blocks])
    return table, ads


@pytest.mark.parametrize("T,in_dim,out_dims,lora", [
    (28, 4096, [4096, 1024, 1024], True),   # QKV with adapters
    (1, 4096, [4096], False),
    (5, 256, [200], True),                  # N not a multiple of 16
    (64, 512, [96, 96], True),              # 4 token tiles
    (17, 14336, [4096], False),             # long K (Down shape)
    (28, 4096, [128256], False),            # LM head: long K-slices (as many steps as the LDS holds)
])
def test_packed_round_matches_row_major_bitwise(dev, T, in_dim, out_dims, lora):
    ops = _ops()
    n = sum(out_dims)
    w = randn((n, in_dim), SEED_W, std=0.02)
    xs = [randn((1, in_dim), SEED_X * 100 + i) for i in range(T)]
    table, ads = _table(dev, in_dim, out_dims, 3) if lora else (None, None)
    ids = [i % 3 for i in range(T)] if lora else None
    kw = dict(seg_lora=ids, table=table, blk_cols=out_dims) if lora else {}
    wd = w.to(dev)
    pw = ops.pack_weight(wd)
    got_rm = [torch.zeros(1, n, dtype=BF16, device=dev) for _ in range(T)]
    got_pk = [torch.zeros(1, n, dtype=BF16, device=dev) for _ in range(T)]
    xd = [x.to(dev) for x in xs]
    ops.round_fused(xd, got_rm, [1] * T, wd, None, **kw)
    ops.round_ex(xd, got_pk, [1] * T, pw, None, **kw)
    torch.cuda.synchronize()
    for i in range(T):
        assert bits_equal(got_pk[i].cpu(), got_rm[i].cpu()), f"token {i}"
    op = {3: ref.OP_QKV_FUSED, 2: ref.OP_GATE_UP_FUSED}.get(len(out_dims), ref.OP_O_PROJ)
    want = ref.round_with_lora(op, xs, [1] * T, w, [ads[j] for j in ids] if lora else [None] * T, out_dims)
    for i in range(T):
        assert_close(got_pk[i].cpu(), want[i], what=f"token {i}")


def _table_packed_a(dev, in_dim, out_dims, ranks, scale=2.0):
    """Two tables with the same adapters: row-major lora_A and fragment-tile
    lora_A (a_layout 1)."""
    ops = _ops()
    t_rm, t_pk, ads = ops.LoraTable(dev), ops.LoraTable(dev), []
    for i, r in enumerate(ranks):
        blocks = [(randn((r, in_dim), 7000 + 10 * i + 2 * j, std=0.02),
                   randn((od, r), 7000 + 10 * i + 2 * j + 1, std=0.02)) for j, od in enumerate(out_dims)]
        A = torch.cat([a for a, _ in blocks], 0).contiguous().to(dev)
        Bs = [b.contiguous().to(dev) for _, b in blocks]
        t_rm.add(A, Bs, r, scale)
        t_pk.add(ops.pack_weight(A), Bs, r, scale)
        ads.append([(a, b, scale) for a, b in blocks])
    return t_rm, t_pk, ads


@pytest.mark.parametrize("T,in_dim,out_dims,ranks,ids", [
    (28, 4096, [4096, 1024, 1024], [16] * 28, list(range(28))),     # config-4 QKV: own adapter per token
    (28, 4096, [4096], [16] * 28, list(range(28))),                 # O
    (28, 4096, [14336, 14336], [16] * 28, list(range(28))),         # Gate+Up
    (28, 14336, [4096], [16] * 28, list(range(28))),                # Down (long K)
    (5, 256, [200], [8, 16], [1, 0, 1, -1, 0]),                     # rank 8 (padded tile), a token without one
    (64, 512, [96, 96], [16, 8, 16], [i % 3 for i in range(64)]),  # four token tiles, shared adapters
])
def test_packed_lora_a_matches_row_major_bitwise(dev, T, in_dim, out_dims, ranks, ids):
    """Rounds whose adapters' stacked lora_A are fragment tiles (a_layout 1)
    equal the same rounds over row-major lora_A bit for bit (the same
    products in the same order), with row-major and with packed weights, and
    match the oracle."""
    ops = _ops()
    n = sum(out_dims)
    w = randn((n, in_dim), SEED_W + 3, std=0.02)
    xs = [randn((1, in_dim), SEED_X * 50 + i) for i in range(T)]
    t_rm, t_pk, ads = _table_packed_a(dev, in_dim, out_dims, ranks)
    wd = w.to(dev)
    pw = ops.pack_weight(wd)
    xd = [x.to(dev) for x in xs]
    outs = {}
    for name, wt, tab in (("rm", pw, t_rm), ("pk", pw, t_pk), ("pk_rowmajor_w", wd, t_pk)):
        y = [torch.zeros(1, n, dtype=BF16, device=dev) for _ in range(T)]
        ops.round_ex(xd, y, [1] * T, wt, None, seg_lora=ids, table=tab, blk_cols=out_dims)
        torch.cuda.synchronize()
        outs[name] = torch.cat([t.cpu() for t in y], 0)
    assert bits_equal(outs["pk"], outs["rm"])
    assert bits_equal(outs["pk_rowmajor_w"], outs["rm"])
    op = {3: ref.OP_QKV_FUSED, 2: ref.OP_GATE_UP_FUSED}.get(len(out_dims), ref.OP_O_PROJ)
    want = ref.round_with_lora(op, xs, [1] * T, w, [ads[j] if j >= 0 else None for j in ids], out_dims)
    for i in range(T):
        assert_close(outs["pk"][i:i + 1], want[i], what=f"token {i}")


def test_packed_lora_a_refused_where_unsupported(dev):
    """Fragment-tile lora_A is read only by the K-sliced decode rounds:
    mixed layouts in one round, the whole-K round, the prefill regime and
    the segmented delta refuse it."""
    ops = _ops()
    t_rm, t_pk, _ = _table_packed_a(dev, 64, [32], [16, 16])
    A = torch.zeros(16, 64, dtype=BF16, device=dev)
    B = torch.zeros(32, 16, dtype=BF16, device=dev)
    t_pk.add(A, [B], 16, 1.0)  # entry 2: row-major in the packed table
    w = randn((32, 64), 5).to(dev)
    x1 = [torch.zeros(1, 64, dtype=BF16, device=dev) for _ in range(3)]
    y1 = [torch.zeros(1, 32, dtype=BF16, device=dev) for _ in range(3)]
    with pytest.raises(ValueError, match="all have row-major or all fragment-tile"):
        ops.round_ex(x1, y1, [1, 1, 1], w, seg_lora=[0, 1, 2], table=t_pk, blk_cols=[32])
    xs = [torch.zeros(65, 64, dtype=BF16, device=dev)]
    ys = [torch.zeros(65, 32, dtype=BF16, device=dev)]
    with pytest.raises(RuntimeError, match="at most 64 token rows"):
        ops.round_ex(xs, ys, [65], w, seg_lora=[0], table=t_pk, blk_cols=[32])
    with pytest.raises(ValueError, match="row-major lora_A"):
        ops.lora_segmented(torch.zeros(2, 64, dtype=BF16, device=dev), [2], [0], t_pk, [32],
                           torch.zeros(2, 32, dtype=BF16, device=dev))
    with pytest.raises(ValueError, match="a_layout"):
        ops.round_fusion(w_layout=2, a_layout=1)
    with pytest.raises(ValueError, match="a_layout 1 needs"):
        ops.round_ex(x1[:1], y1[:1], [1], w, seg_lora=[0], table=t_rm, blk_cols=[32],
                     fusion=ops.round_fusion(a_layout=1))


def test_packed_round_with_norm_and_residual_fusions(dev):
    """Fused forms over packed weights equal the same fusions over row-major
    weights bit for bit."""
    ops = _ops()
    H, T = 4096, 28
    w = randn((H, H), SEED_W + 1, std=0.02)
    gamma = (1 + randn((H,), 77, std=0.1).float()).to(BF16).to(dev)
    hs = torch.cat([randn((1, H), SEED_X + i, std=3.0) for i in range(T)], 0).to(dev)
    ss = torch.stack([hs.float()[:, j:j + 256].pow(2).sum(1) for j in range(0, H, 256)], 1).contiguous()
    wd = w.to(dev)
    pw = ops.pack_weight(wd)
    outs = []
    for wt, layout in ((wd, 0), (pw, 1)):
        h2 = hs.clone()
        ss_out = torch.zeros(T, 16, dtype=torch.float32, device=dev)
        y = [torch.zeros(1, H, dtype=BF16, device=dev) for _ in range(T)]
        ops.round_ex([hs[i:i + 1] for i in range(T)], y, [1] * T, wt, None,
                     fusion=ops.round_fusion(norm_weight=gamma, eps=1e-5, ss_in=ss, w_layout=layout))
        ops.round_ex([y[i] for i in range(T)], [h2[i:i + 1] for i in range(T)], [1] * T, wt, None,
                     fusion=ops.round_fusion(out_mode=1, ss_out=ss_out, w_layout=layout))
        torch.cuda.synchronize()
        outs.append((torch.cat(y, 0).cpu(), h2.cpu(), ss_out.cpu()))
    assert bits_equal(outs[0][0], outs[1][0])
    assert bits_equal(outs[0][1], outs[1][1])
    assert torch.equal(outs[0][2], outs[1][2])


@pytest.mark.parametrize("T", [28, 64])
def test_norm_fused_lm_head_packed_matches_row_major_and_oracle(dev, T):
    """The decode step's LM-head round: vocab 128256, the final RMSNorm on
    the staged residual rows (norm_weight + ss_in), long K-slices whose LDS
    holds the slice, gamma and the row factors.  T = 64 runs four token
    tiles.  Packed equals row-major bit for bit; sampled rows match the
    oracle's rms_norm -> x @ W^T."""
    ops = _ops()
    H, V, eps = 4096, 128256, 1e-5
    g = torch.Generator(device=dev).manual_seed(SEED_W + T)
    wd = (torch.randn(V, H, generator=g, device=dev) * 0.02).to(BF16)
    gamma = (1 + randn((H,), 78, std=0.1).float()).to(BF16)
    hs = torch.cat([randn((1, H), SEED_X + 300 + i, std=3.0) for i in range(T)], 0)
    ss = torch.stack([hs.float()[:, j:j + 256].pow(2).sum(1) for j in range(0, H, 256)], 1).contiguous()
    hd, gd, ssd = hs.to(dev), gamma.to(dev), ss.to(dev)
    pw = ops.pack_weight(wd)
    outs = []
    for wt, layout in ((wd, 0), (pw, 1)):
        y = torch.zeros(T, V, dtype=BF16, device=dev)
        ops.round_ex([hd[i:i + 1] for i in range(T)], [y[i:i + 1] for i in range(T)], [1] * T, wt, None,
                     fusion=ops.round_fusion(norm_weight=gd, eps=eps, ss_in=ssd, w_layout=layout))
        torch.cuda.synchronize()
        outs.append(y.cpu())
    assert bits_equal(outs[0], outs[1])
    rows = [0, T // 2 + 1, T - 1]
    w = wd.cpu()
    want = ref.base_gemm(ref.rms_norm(hs[rows], gamma, eps), w)
    assert_close(outs[1][rows], want, what=f"LM head T={T}")


def test_packed_weight_rejected_where_unsupported(dev):
    ops = _ops()
    w = randn((64, 64), 5).to(dev)
    pw = ops.pack_weight(w)
    xs = [torch.zeros(65, 64, dtype=BF16, device=dev)]
    ys = [torch.zeros(65, 64, dtype=BF16, device=dev)]
    with pytest.raises(RuntimeError, match="at most 64 token rows"):
        ops.round_ex(xs, ys, [65], pw)
    with pytest.raises(ValueError, match="PackedWeight"):
        ops.round_ex(xs, ys, [1], w, fusion=ops.round_fusion(w_layout=1))
    with pytest.raises(ValueError, match="multiple of 32"):
        ops.pack_weight(torch.zeros(16, 48, dtype=BF16, device=dev))
