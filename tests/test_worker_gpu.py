"""GPU parity of the worker-side classes (FusedLoRA, SyncRemoteLoRALinear,
PagedKVCache, batch_flash_attention) against the CPU oracle."""

import math

import pytest
import torch

from oracle import reference_path as ref
from tests._util import BF16, assert_close, bits_equal, randn

pytestmark = pytest.mark.gpu


def _mods(r, in_dim, out_dims, s, seed):
    from swarmlora_amd.worker.model_builder import FastLoRAModule
    host = [(randn((r, in_dim), seed + 2 * i, std=0.02), randn((o, r), seed + 2 * i + 1, std=0.02))
            for i, o in enumerate(out_dims)]
    return host, [FastLoRAModule(A.cuda(), B.cuda(), s) for A, B in host]


@pytest.mark.parametrize("t", [1, 16])
def test_fused_lora_qkv_matches_oracle(dev, t):
    from swarmlora_amd.worker.model_builder import FusedLoRA
    dims = [4096, 1024, 1024]
    host, mods = _mods(16, 4096, dims, 2.0, seed=100)
    fl = FusedLoRA(mods, dims, dev, BF16)
    x = randn((1, t, 4096), 7)
    got = fl(x.to(dev))
    torch.cuda.synchronize()
    fA, fB = ref.fused_lora_weights([(A, B, 2.0) for A, B in host], dims)
    want = ref.fused_lora_forward(x, fA, fB, dims)
    for g, w in zip(got, want):
        assert g.shape == w.shape
        assert_close(g, w, what="fused lora")


def test_fused_lora_missing_module_and_no_lora(dev):
    from swarmlora_amd.worker.model_builder import FusedLoRA
    dims = [512, 128, 128]
    host, mods = _mods(8, 512, dims, 1.0, seed=5)
    mods[1] = None
    fl = FusedLoRA(mods, dims, dev, BF16)
    d = fl(randn((1, 3, 512), 1).to(dev))
    assert float(d[1].abs().max()) == 0.0 and float(d[0].abs().max()) > 0
    empty = FusedLoRA([None, None], [4, 4], dev, BF16)
    assert not empty.has_lora and empty(randn((1, 1, 4), 0).to(dev)) == [None, None]


@pytest.mark.parametrize("in_dim", [4096, 14336])
def test_remote_lora_delta_matches_oracle(dev, in_dim):
    from swarmlora_amd.worker.model_builder import SyncRemoteLoRALinear
    host, mods = _mods(16, in_dim, [4096], 2.0, seed=33)
    m = SyncRemoteLoRALinear(3, 0, 4096, mods[0])
    x = randn((1, 2, in_dim), 3)
    got = m.delta(x.to(dev))
    torch.cuda.synchronize()
    A, B = host[0]
    assert_close(got, ref.remote_lora_delta(x, A, B, 2.0), what="remote lora")


@pytest.mark.parametrize("m,rank,nblk,in_dim,kmajor", [
    (1, 16, 3, 4096, True),    # FusedLoRA QKV: fused_A [k, 48], 16-byte loads over j
    (4, 16, 2, 4096, True),    # FusedLoRA Gate+Up shape, four rows
    (3, 4, 3, 512, True),      # nr = 12: scalar loads of fused_A
    (2, 32, 2, 4096, True),    # nr = 64
    (1, 16, 1, 14336, False),  # SyncRemoteLoRALinear Down: lora_A [16, k], lora_B [4096, 16]
    (4, 8, 1, 4096, False),
])
def test_lora_rows_matches_oracle(dev, m, rank, nblk, in_dim, kmajor):
    """ops.lora_rows (one launch) against the oracle's two bf16 products, for
    the fused (block-diagonal fused_B) and the per-projection (lora_B) forms."""
    from swarmlora_amd import ops
    widths = [4096, 1024, 1024][:nblk] if nblk > 1 else [4096]
    host = [(randn((rank, in_dim), 50 + i, std=0.02), randn((w, rank), 60 + i, std=0.02)) for i, w in enumerate(widths)]
    x = randn((m, in_dim), 9)
    if kmajor:
        fA, fB = ref.fused_lora_weights([(A, B, 2.0) for A, B in host], widths)
        blocks, col = [], 0
        fBd = fB.to(dev)
        for i, w in enumerate(widths):
            blocks.append((fBd[i * rank:(i + 1) * rank, col:col + w], w, True))
            col += w
        got = ops.lora_rows(x.to(dev), fA.to(dev), True, blocks, rank)
        want = torch.cat(ref.fused_lora_forward(x, fA, fB, widths), -1)
    else:
        A, B = host[0]
        got = ops.lora_rows(x.to(dev), A.to(dev), False, [(B.to(dev), B.shape[0], False)], rank, 2.0)
        want = ref.remote_lora_delta(x, A, B, 2.0)
    torch.cuda.synchronize()
    assert got.shape == want.shape
    assert_close(got, want, what="lora_rows")


def test_lora_rows_rejects_what_it_cannot_do(dev):
    from swarmlora_amd import ops
    x = torch.zeros(5, 512, dtype=BF16, device=dev)
    A = torch.zeros(16, 512, dtype=BF16, device=dev)
    B = torch.zeros(64, 16, dtype=BF16, device=dev)
    with pytest.raises(RuntimeError, match="at most 4 rows"):
        ops.lora_rows(x, A, False, [(B, 64, False)], 16)
    with pytest.raises(RuntimeError, match="shrink columns"):
        ops.lora_rows(x[:1], torch.zeros(80, 512, dtype=BF16, device=dev), False, [(B, 64, False)], 16)


def test_paged_kv_cache_allocation_and_zeroing(dev):
    from swarmlora_amd.worker.paged_attention import PagedKVCache
    c = PagedKVCache(2, 8, 128, 16, 2, 64, dev, BF16)
    o = ref.PagedKVCacheRef(16, 2, 64)
    for sid, n in ((0, 17), (1, 1), (0, 33)):
        c.ensure_blocks_for_length(sid, n)
        o.ensure_blocks_for_length(sid, n)
    assert c.slot_block_tables == o.slot_block_tables
    bt = c.get_block_table_tensor([0, 1]).cpu()
    assert bt.dtype == torch.int32 and bt[0, :3].tolist() == [0, 1, 3] and bt[1, 0] == 2 and bt[1, 1] == 0
    for kc in c.key_caches + c.value_caches:
        kc.fill_(1.0)
    c.free_slot(0)
    torch.cuda.synchronize()
    for kc in c.key_caches + c.value_caches:
        assert float(kc[[0, 1, 3]].abs().max()) == 0.0
        assert float(kc[2].min()) == 1.0
    assert c.free_blocks[-3:] == [0, 1, 3]


def test_cos_sin_cache_matches_oracle(dev):
    from swarmlora_amd.worker.paged_attention import RotaryInvFreq, build_vllm_cos_sin_cache
    cs = build_vllm_cos_sin_cache(RotaryInvFreq(128, 500000.0), 2048, dev, BF16)
    want = ref.cos_sin_cache(ref.rope_inv_freq(128, 500000.0), 2048)
    assert_close(cs, want, tol=1e-2, what="cos_sin")


@pytest.mark.parametrize("q_len,ctx0", [(1, [37]), (16, [32])])
def test_batch_flash_attention_matches_oracle(dev, q_len, ctx0):
    """Through PagedKVCache + the fused-QKV views a worker gets from
    get_outputs_slot (q/k/v read in place with a 6144-element token stride)."""
    from swarmlora_amd.worker.batched_ops import WorkerBatchedOps
    from swarmlora_amd.worker.paged_attention import PagedKVCache, RotaryInvFreq, build_vllm_cos_sin_cache
    H, KV, D = 32, 8, 128
    c = PagedKVCache(1, KV, D, 16, 1, 256, dev, BF16)
    sid = 0
    c.ensure_blocks_for_length(sid, ctx0[0] + q_len)
    c.slot_seq_lens[sid] = ctx0[0]
    hist_k = randn(c.key_caches[0].shape, 40)
    hist_v = randn(c.value_caches[0].shape, 41)
    c.key_caches[0].copy_(hist_k)
    c.value_caches[0].copy_(hist_v)
    fused = randn((1, q_len, H * D + 2 * KV * D), 42)
    qkv = list(fused.to(dev).split([H * D, KV * D, KV * D], dim=-1))
    cs = build_vllm_cos_sin_cache(RotaryInvFreq(D, 500000.0), 256, dev, BF16)
    seqlens = c.get_seq_lens_tensor([sid])
    positions = (seqlens.long().unsqueeze(1) + torch.arange(q_len, device=dev).unsqueeze(0)).reshape(-1)
    meta = {"cache_seqlens": seqlens, "block_tables": c.get_block_table_tensor([sid]), "positions": positions,
            "bufs_q": torch.empty(1, q_len, H, D, device=dev)}
    out = WorkerBatchedOps.batch_flash_attention([sid], {sid: tuple(qkv)}, c, cs, 0, H, KV, D, meta)[sid]
    torch.cuda.synchronize()
    q, k, v = [p.reshape(1, q_len, h, D) for p, h in zip(fused.split([H * D, KV * D, KV * D], -1), (H, KV, KV))]
    kc, vc = hist_k.clone(), hist_v.clone()
    want, _, _ = ref.paged_attention(q, k, v, kc, vc, meta["block_tables"].cpu(), seqlens.cpu(), positions.cpu(),
                                     cs.cpu(), 1 / math.sqrt(D))
    assert out.shape == (1, q_len, H * D)
    assert_close(out, want, what="batch_flash_attention")
    assert bits_equal(c.value_caches[0], vc)
