"""GPU tests of the segmented LoRA delta (swl_lora_segmented_bf16) against
the oracle's per-slot delta of the reference (FusedLoRA.forward for fused
projections, SyncRemoteLoRALinear for single ones: model_builder.py:193-262),
for decode-shaped (one row per segment) and prefill-shaped (ragged) batches,
mixed ranks, segments without an adapter, and both the write and the add
forms; the add form against the base output plus the delta."""

import pytest
import torch

from oracle import reference_path as ref
from tests._util import BF16, assert_close, bits_equal, randn

pytestmark = pytest.mark.gpu


def _ops():
    from swarmlora_amd import ops
    return ops


def _case(dev, rows, ranks, k, dims, seed):
    ops = _ops()
    table = ops.LoraTable(dev)
    ads = []
    for i, r in enumerate(ranks):
        if r is None:
            ads.append(None)
            continue
        blocks = [(randn((r, k), seed * 100 + 10 * i + 2 * j, std=0.05),
                   randn((d, r), seed * 100 + 10 * i + 2 * j + 1, std=0.05)) for j, d in enumerate(dims)]
        table.add(torch.cat([A for A, _ in blocks], 0).contiguous().to(dev), [B.contiguous().to(dev) for _, B in blocks],
                  r, 1.5)
        ads.append([(A, B, 1.5) for A, B in blocks])
    idx, e = [], 0
    for r in ranks:
        idx.append(-1 if r is None else e)
        e += r is not None
    xs = [randn((t, k), seed + 7 * i) for i, t in enumerate(rows)]
    return table, ads, idx, xs


def _want(ads, xs, dims):
    out = []
    for ad, x in zip(ads, xs):
        if x.shape[0] == 0:
            continue
        if ad is None:
            out.append(torch.zeros(x.shape[0], sum(dims)))
        elif len(dims) > 1:
            fA, fB = ref.fused_lora_weights(ad, dims)
            out.append(torch.cat(ref.fused_lora_forward(x, fA, fB, dims), -1).float())
        else:
            A, B, s = ad[0]
            out.append(ref.remote_lora_delta(x, A, B, s).float())
    return torch.cat(out, 0)


@pytest.mark.parametrize("rows,ranks,k,dims", [
    ([1] * 28, [16] * 28, 4096, [4096, 1024, 1024]),                 # decode QKV, one adapter per row
    ([1, 1, 1, 1, 1], [8, None, 64, 16, 8], 4096, [4096]),            # O-shaped, a row without adapter
    ([37, 0, 130, 5], [32, 16, None, 4], 1024, [512, 512]),           # ragged prefill, empty segment
    ([70, 3], [64, 64], 14336, [4096]),                              # long K (Down)
])
def test_delta_matches_oracle(dev, rows, ranks, k, dims):
    ops = _ops()
    table, ads, idx, xs = _case(dev, rows, ranks, k, dims, seed=3)
    x = torch.cat(xs, 0).to(dev)
    y = torch.full((x.shape[0], sum(dims)), 7.0, dtype=BF16, device=dev)
    ops.lora_segmented(x, rows, idx, table, dims, y, add=False)
    torch.cuda.synchronize()
    want = _want(ads, xs, dims)
    assert_close(y.cpu(), want, what="delta")
    # rows without an adapter are written as exact zeros
    off = 0
    for t, r in zip(rows, ranks):
        if r is None and t > 0:
            assert bits_equal(y[off:off + t].cpu(), torch.zeros(t, sum(dims), dtype=BF16))
        off += t


def test_add_form_is_base_plus_delta(dev):
    ops = _ops()
    rows, ranks, k, dims = [4, 9, 2], [16, None, 8], 2048, [2048]
    table, ads, idx, xs = _case(dev, rows, ranks, k, dims, seed=11)
    x = torch.cat(xs, 0).to(dev)
    base = randn((x.shape[0], sum(dims)), 99)
    y = base.clone().to(dev)
    ops.lora_segmented(x, rows, idx, table, dims, y, add=True)
    torch.cuda.synchronize()
    want = base.float() + _want(ads, xs, dims)
    assert_close(y.cpu(), want, what="y + delta")
    # the segment without an adapter is untouched
    assert bits_equal(y[4:13].cpu(), base[4:13])


def test_rejects_bad_arguments(dev):
    ops = _ops()
    table, ads, idx, xs = _case(dev, [2], [8], 64, [64], seed=5)
    x = torch.cat(xs, 0).to(dev)
    y = torch.zeros(2, 64, dtype=BF16, device=dev)
    with pytest.raises(RuntimeError, match="sum to N"):
        ops.lora_segmented(x, [2], idx, table, [32], y)
    with pytest.raises(ValueError, match="sum\\(seg_rows\\)"):
        ops.lora_segmented(x, [3], idx, table, [64], y)
