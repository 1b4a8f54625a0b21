"""GPU tests of the allocation-free round entry point
(swl_round_ex_noalloc_bf16, include/swl.h), called through the C ABI.

It runs the same kernels as swl_round_ex_bf16 with the K-slice partials in
the library's fixed device array instead of the growable scratch, so its
outputs must equal swl_round_ex_bf16's bit for bit: on two calls in a row
(the second with fewer token rows, so it runs over what the first left in
the array), replayed from a HIP graph captured around it (the use it is
for), and it must refuse what does not fit.
"""

import pytest
import torch

from tests._util import BF16, SEED_W, SEED_X, bits_equal, randn

pytestmark = pytest.mark.gpu

H, I, R = 4096, 14336, 16


def _ops():
    from swarmlora_amd import ops
    return ops


def _gate_up(dev):
    """Packed Gate+Up weight, a LoRA table of 3 adapters (gate / up blocks),
    the post-attention norm weight."""
    ops = _ops()
    w = randn((2 * I, H), SEED_W + 40, std=0.02)
    table = ops.LoraTable(dev)
    for i in range(3):
        blocks = [(randn((R, H), 7000 + 4 * i + 2 * j, std=0.02), randn((I, R), 7001 + 4 * i + 2 * j, std=0.02))
                  for j in range(2)]
        table.add(torch.cat([a for a, _ in blocks], 0).to(dev), [b.to(dev) for _, b in blocks], R, 2.0)
    gamma = (1 + randn((H,), 41, std=0.1).float()).to(BF16)
    return ops.pack_weight(w.to(dev)), table, gamma


def _inputs(T, seed, dev):
    hs = torch.cat([randn((1, H), seed + i, std=2.0) for i in range(T)], 0)
    ss = torch.stack([hs.float()[:, j:j + 256].pow(2).sum(1) for j in range(0, H, 256)], 1).contiguous()
    return hs.to(dev), ss.to(dev)


def _run(pw, table, gamma_d, hd, ssd, T, noalloc, out=None):
    ops = _ops()
    out = torch.zeros(T, I, dtype=BF16, device=hd.device) if out is None else out
    ops.round_ex([hd[i:i + 1] for i in range(T)], [out[i:i + 1] for i in range(T)], [1] * T, pw, None,
                 seg_lora=[i % 3 for i in range(T)], table=table, blk_cols=[I, I],
                 fusion=ops.round_fusion(norm_weight=gamma_d, eps=1e-5, ss_in=ssd, out_mode=2), noalloc=noalloc)
    return out


def test_noalloc_round_equals_round_ex_on_two_calls_in_a_row(dev):
    """Gate+Up round at 8B widths (norm on staging, pooled rank-16 adapters,
    SiLU*up epilogue, packed weight): 28 token rows, then 5."""
    pw, table, gamma = _gate_up(dev)
    gd = gamma.to(dev)
    a_d, a_ss = _inputs(28, SEED_X + 500, dev)
    b_d, b_ss = _inputs(5, SEED_X + 600, dev)
    want_a = _run(pw, table, gd, a_d, a_ss, 28, noalloc=False)
    want_b = _run(pw, table, gd, b_d, b_ss, 5, noalloc=False)
    torch.cuda.synchronize()
    got_a = _run(pw, table, gd, a_d, a_ss, 28, noalloc=True)
    got_b = _run(pw, table, gd, b_d, b_ss, 5, noalloc=True)
    torch.cuda.synchronize()
    assert bits_equal(got_a.cpu(), want_a.cpu())
    assert bits_equal(got_b.cpu(), want_b.cpu())


def test_noalloc_round_replays_from_a_captured_graph(dev):
    """The round captured into a HIP graph without any earlier call of its
    shape (nothing sized beforehand), replayed three times over new inputs
    with eager work and synchronisation between replays; every replay equals
    an eager swl_round_ex_bf16 of the same inputs bit for bit."""
    ops = _ops()
    T = 12
    w = randn((H, H), SEED_W + 41, std=0.02)
    pw = ops.pack_weight(w.to(dev))
    x_static = torch.zeros(T, H, dtype=BF16, device=dev)
    y_static = torch.zeros(T, H, dtype=BF16, device=dev)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ops.round_ex([x_static[i:i + 1] for i in range(T)], [y_static[i:i + 1] for i in range(T)], [1] * T, pw,
                         noalloc=True)
    torch.cuda.synchronize()
    for rep in range(3):
        x = randn((T, H), SEED_X + 700 + rep).to(dev)
        x_static.copy_(x)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = torch.zeros(T, H, dtype=BF16, device=dev)
        ops.round_ex([x[i:i + 1] for i in range(T)], [want[i:i + 1] for i in range(T)], [1] * T, pw)
        torch.cuda.synchronize()
        assert bits_equal(y_static.cpu(), want.cpu()), f"replay {rep}"


def test_noalloc_round_refuses_what_does_not_fit(dev):
    ops = _ops()
    w = torch.zeros(64, 4096, dtype=BF16, device=dev)
    xs = [torch.zeros(65, 4096, dtype=BF16, device=dev)]
    ys = [torch.zeros(65, 64, dtype=BF16, device=dev)]
    with pytest.raises(RuntimeError, match="at most 64 token rows"):
        ops.round_ex(xs, ys, [65], w, noalloc=True)
    # partials of 64 rows x 131072 columns (at least 4 K-slices of fp32: 128 MiB) do not fit the
    # 64 MiB array: refused.  Every buffer is really allocated at its full size (a 1 GiB weight), so
    # the call stays in bounds whatever order the checks run in.
    n = 131072
    w = torch.zeros(n, 4096, dtype=BF16, device=dev)
    xs = [torch.zeros(64, 4096, dtype=BF16, device=dev)]
    ys = [torch.zeros(64, n, dtype=BF16, device=dev)]
    with pytest.raises(RuntimeError, match="allocation-free scratch"):
        ops.round_ex(xs, ys, [64], w, noalloc=True)
    del w
