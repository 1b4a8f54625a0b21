"""GPU parity of the worker-side token-row kernels (RMSNorm with the residual
add, SiLU*up, paged attention over per-token rows) against the CPU oracle.

Rows live in separate buffers (as slot buffers do), so every test scatters
its tokens over distinct allocations.
"""

import math

import pytest
import torch

from oracle import reference_path as ref
from tests._util import BF16, assert_close, bits_equal, randn

pytestmark = pytest.mark.gpu


def _ops():
    from swarmlora_amd import ops
    return ops


def _rows(dev, n, width, fill=0.0):
    """n separate buffers (slot-like), each with a little slack after the row."""
    return [torch.full((width + 64,), fill, dtype=BF16, device=dev) for _ in range(n)]


@pytest.mark.parametrize("ntok,d", [(1, 4096), (28, 4096), (64, 512), (3, 8)])
def test_rmsnorm_rows_no_add(dev, ntok, d):
    ops = _ops()
    h = randn((ntok, d), 1)
    w = (1 + randn((d,), 2, std=0.1).float()).to(BF16)
    outs = _rows(dev, ntok, d, fill=-3.0)
    hd = h.to(dev)
    ops.rmsnorm_rows(hd, w.to(dev), 1e-5, [o[:d] for o in outs])
    torch.cuda.synchronize()
    want = ref.rms_norm(h, w, 1e-5)
    got = torch.stack([o[:d].cpu() for o in outs])
    assert_close(got, want, what="rmsnorm")
    assert bits_equal(hd, h), "h must be unchanged without add_rows"
    for o in outs:
        assert bool((o[d:] == -3.0).all()), "row tail must be untouched"


@pytest.mark.parametrize("ntok,d", [(28, 4096), (5, 1024)])
def test_rmsnorm_rows_residual_add(dev, ntok, d):
    """h = residual + result (one bf16 rounding), then RMSNorm of the sum."""
    ops = _ops()
    h = randn((ntok, d), 3)
    add = randn((ntok, d), 4, std=0.5)
    w = (1 + randn((d,), 5, std=0.1).float()).to(BF16)
    adds = _rows(dev, ntok, d)
    for a, r in zip(adds, add):
        a[:d].copy_(r)
    outs = _rows(dev, ntok, d)
    hd = h.to(dev)
    ops.rmsnorm_rows(hd, w.to(dev), 1e-5, [o[:d] for o in outs], add_rows=[a[:d] for a in adds])
    torch.cuda.synchronize()
    hsum = h + add
    assert bits_equal(hd, hsum), "residual add must be bit-exact bf16 addition"
    assert_close(torch.stack([o[:d].cpu() for o in outs]), ref.rms_norm(hsum, w, 1e-5), what="rmsnorm(add)")


def test_rmsnorm_rows_constant_row_is_weight(dev):
    """Closed form: a row of equal values c has rms |c|, so with eps = 0 the
    normalised row is sign(c) and the output equals +-weight."""
    ops = _ops()
    d = 4096
    h = torch.full((2, d), 0.75, dtype=BF16)
    h[1] = -2.0
    w = randn((d,), 9)
    outs = _rows(dev, 2, d)
    ops.rmsnorm_rows(h.to(dev), w.to(dev), 0.0, [o[:d] for o in outs])
    torch.cuda.synchronize()
    assert bits_equal(outs[0][:d], w)
    assert bits_equal(outs[1][:d], -w)


@pytest.mark.parametrize("ntok,inter", [(1, 14336), (28, 14336), (7, 64)])
def test_silu_mul_rows(dev, ntok, inter):
    ops = _ops()
    gu = randn((ntok, 2 * inter), 6, std=2.0)
    ins = _rows(dev, ntok, 2 * inter)
    for b, r in zip(ins, gu):
        b[:2 * inter].copy_(r)
    outs = _rows(dev, ntok, inter, fill=5.0)
    ops.silu_mul_rows([b[:2 * inter] for b in ins], [o[:inter] for o in outs], inter)
    torch.cuda.synchronize()
    want = ref.silu_mul(gu[:, :inter], gu[:, inter:])
    assert_close(torch.stack([o[:inter].cpu() for o in outs]), want, what="silu*up")
    for o in outs:
        assert bool((o[inter:] == 5.0).all())


def test_silu_mul_rows_zero_gate_is_zero(dev):
    """silu(0) = 0 exactly, whatever up is."""
    ops = _ops()
    inter = 256
    b = torch.zeros(2 * inter, dtype=BF16, device=dev)
    b[inter:] = randn((inter,), 1).to(dev)
    o = torch.ones(inter, dtype=BF16, device=dev)
    ops.silu_mul_rows([b], [o], inter)
    torch.cuda.synchronize()
    assert float(o.abs().max()) == 0.0


@pytest.mark.parametrize("nseq,L,ctx0", [(4, 1, [127, 128, 1000, 2047]), (2, 3, [5, 40]), (28, 1, None)])
def test_paged_attention_rows_matches_strided(dev, nseq, L, ctx0):
    """Row mode reads q/k/v from separate fused rows and writes separate
    output rows: it must give the strided entry point's bits and match the
    oracle."""
    ops = _ops()
    hq, hkv, d, bs = 32, 8, 128, 16
    if ctx0 is None:
        g = torch.Generator().manual_seed(3)
        ctx0 = torch.randint(128, 2049, (nseq,), generator=g).tolist()
    max_blocks = (max(ctx0) + L + bs - 1) // bs
    nb = nseq * max_blocks + 2
    g = torch.Generator().manual_seed(11)
    bt = torch.randperm(nb, generator=g)[: nseq * max_blocks].reshape(nseq, max_blocks).to(torch.int32)
    kc = randn((nb, bs, hkv, d), 12)
    vc = randn((nb, bs, hkv, d), 13)
    fused = randn((nseq * L, (hq + 2 * hkv) * d), 14)
    sl = torch.tensor(ctx0, dtype=torch.int32)
    pos = (sl.long().unsqueeze(1) + torch.arange(L).unsqueeze(0)).reshape(-1)
    cs = ref.cos_sin_cache(ref.rope_inv_freq(d, 500000.0), 4096)
    scale = 1 / math.sqrt(d)
    W = (hq + 2 * hkv) * d

    # row mode over separate buffers
    qkv_bufs = _rows(dev, nseq * L, W)
    for b, r in zip(qkv_bufs, fused):
        b[:W].copy_(r)
    out_bufs = _rows(dev, nseq * L, hq * d, fill=9.0)
    kc1, vc1 = kc.to(dev), vc.to(dev)
    ops.paged_attention_rows([b[:W] for b in qkv_bufs], [o[:hq * d] for o in out_bufs], L, hq, hkv, d, kc1, vc1,
                             bt.to(dev), sl.to(dev), pos.to(dev), cs.to(dev), scale)
    # strided entry point on the same inputs
    fd = fused.to(dev).reshape(nseq, L, W)
    q, k, v = fd.split([hq * d, hkv * d, hkv * d], -1)
    kc2, vc2 = kc.to(dev), vc.to(dev)
    out2 = ops.paged_attention(q.reshape(nseq, L, hq, d), k.reshape(nseq, L, hkv, d), v.reshape(nseq, L, hkv, d),
                               kc2, vc2, bt.to(dev), sl.to(dev), pos.to(dev), cs.to(dev), scale)
    torch.cuda.synchronize()
    got = torch.stack([o[:hq * d].cpu() for o in out_bufs]).reshape(nseq, L, hq * d)
    assert bits_equal(got, out2)
    assert bits_equal(kc1, kc2) and bits_equal(vc1, vc2)
    for o in out_bufs:
        assert bool((o[hq * d:] == 9.0).all())
    fr = fused.reshape(nseq, L, W)
    qr, kr, vr = fr.split([hq * d, hkv * d, hkv * d], -1)
    kcr, vcr = kc.clone(), vc.clone()
    want, q_rot, _ = ref.paged_attention(qr.reshape(nseq, L, hq, d), kr.reshape(nseq, L, hkv, d),
                                         vr.reshape(nseq, L, hkv, d), kcr, vcr, bt, sl, pos, cs, scale)
    assert_close(got, want, what="attention rows")
    assert bits_equal(vc1, vcr)
    rot_q = torch.stack([b[:hq * d].cpu() for b in qkv_bufs]).reshape(nseq, L, hq, d)
    assert_close(rot_q, q_rot, what="rope q in place")


def test_row_ops_reject_bad_rows(dev):
    ops = _ops()
    h = torch.zeros(2, 64, dtype=BF16, device=dev)
    w = torch.ones(64, dtype=BF16, device=dev)
    with pytest.raises(ValueError):
        ops.rmsnorm_rows(h, w, 1e-5, [torch.zeros(64, dtype=BF16, device=dev)])  # one row for two tokens
    with pytest.raises(ValueError):
        ops.rmsnorm_rows(h, w, 1e-5, [torch.zeros(32, dtype=BF16, device=dev)] * 2)  # too narrow
    big = torch.zeros(200, dtype=BF16, device=dev)
    with pytest.raises(ValueError):
        ops.silu_mul_rows([big[1:129]], [big[:64]], 64)  # misaligned row
    with pytest.raises(ValueError):
        ops.silu_mul_rows([big] * 65, [big] * 65, 64)  # more than 64 rows


@pytest.mark.parametrize("shape", [(1, 1, 4096), (1, 150, 512), (2, 70, 64)])
def test_rms_norm_matrix_matches_row_kernel(dev, shape):
    """ops.rms_norm (the worker engine's norm) over [b, t, d] in 64-row
    launches: every row equals the oracle, and rows past the first launch
    equal what the row kernel gives for them alone."""
    ops = _ops()
    d = shape[-1]
    x = randn(shape, 11)
    w = (1 + randn((d,), 12, std=0.1).float()).to(BF16)
    got = ops.rms_norm(x.to(dev), w.to(dev), 1e-5)
    torch.cuda.synchronize()
    assert got.shape == x.shape
    assert_close(got.cpu(), ref.rms_norm(x, w, 1e-5), what="rms_norm")
    flat = x.reshape(-1, d)
    n = flat.shape[0]
    tail = list(range(max(0, n - 3), n))
    outs = _rows(dev, len(tail), d)
    ops.rmsnorm_rows(flat[tail].to(dev).contiguous(), w.to(dev), 1e-5, [o[:d] for o in outs])
    torch.cuda.synchronize()
    for o, t in zip(outs, tail):
        assert bits_equal(o[:d], got.reshape(-1, d)[t])


@pytest.mark.parametrize("t,inter", [(1, 14336), (130, 96)])
def test_engine_silu_mul_reads_fused_halves(dev, t, inter):
    """The worker engine's SiLU*up: g and u as the two halves of one Gate+Up
    output (read in place, no copy) and as separate tensors (concatenated
    first) give the same bits, equal to the oracle within tolerance."""
    from swarmlora_amd.worker.engine import silu_mul
    gu = randn((1, t, 2 * inter), 13, std=2.0).to(dev)
    g, u = gu.split([inter, inter], -1)
    a = silu_mul(g, u)
    b = silu_mul(g.clone(), u.clone())
    torch.cuda.synchronize()
    assert bits_equal(a, b)
    want = ref.silu_mul(gu[..., :inter].cpu(), gu[..., inter:].cpu())
    assert_close(a.cpu(), want, what="engine silu*up")
