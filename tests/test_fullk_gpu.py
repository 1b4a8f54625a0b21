"""GPU tests of the whole-K decode round (w_layout 2, fullk_kernel, the
decode step's LM head): one launch per round after the small LoRA shrink
kernel, each workgroup holding the whole K range of the token rows and
finishing its weight tiles (bias, LoRA expand) without partial sums in
memory.

Each case runs the same round through the K-sliced path (w_layout 1, split
and epilogue kernels, tested against the oracle elsewhere) and through the
whole-K path, on the same seeded inputs: the sums run in a different order,
so outputs agree to the bf16 rounding of their last step (normalised max
error well under 1e-2, measured ~4e-3 at most); each is also checked against
the CPU oracle at 1e-2.  Repeated launches, graph replays and the argument
checks are covered too.
"""

import pytest
import torch

from oracle import reference_path as ref
from tests._util import BF16, SEED_A, SEED_W, SEED_X, assert_close, bits_equal, randn, rel_err

pytestmark = pytest.mark.gpu

H, KV, HQ, HD = 4096, 8, 32, 128
EPS = 1e-5
AGREE = 5e-3  # whole-K vs K-sliced (one bf16 rounding apart)


def _ops():
    from swarmlora_amd import ops
    return ops


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
    pw = ops.pack_weight(w_rows.to(dev))
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
    ss = torch.zeros(1, 16, dtype=torch.float32, device=dev)
    with pytest.raises(ValueError, match="out_mode 0 only"):
        ops.round_ex(x33[:1], y33[:1], [1], w, None, fusion=ops.round_fusion(w_layout=2, out_mode=1, ss_out=ss))
