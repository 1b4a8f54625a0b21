"""GPU tests of the QKV round finished inside the attention kernel (round
fusion out_mode 4 + swl_paged_attention_rows_ex_bf16 with rope 3).

The deferred path computes q, k and v from the round's K-slice partials in
the attention kernel's prologue (bias, LoRA expand, RoPE, the new key's KV
append) instead of an epilogue kernel.  It is checked against the same
round with the epilogue (out_mode 3, the RoPE + append fusion already
checked against the oracle in test_fusion_gpu.py) followed by the attention
over the appended pages (rope 2): the appended k / v rows agree within two
bf16 steps at each head row's scale (the K-slice partials are summed in
another order), every
other page entry is untouched, and the attention outputs agree within the
1e-2 bar; the attention output is also checked against the oracle's
paged_attention over the deferred path's own pages.
"""

import math

import pytest
import torch

from oracle import reference_path as ref
from tests._util import BF16, SEED_X, assert_close, randn

pytestmark = pytest.mark.gpu


def _ops():
    from swarmlora_amd import ops
    return ops


@pytest.mark.parametrize("T,bs,lora,ctx_hi", [
    (28, 16, True, 2048),    # config-4 shape: 28 workers, own rank-16 adapters, 1..9 parts
    (5, 32, True, 300),      # pages of 32 keys, short contexts (a single part for some)
    (3, 16, False, 40),      # no adapters, one tile
])
def test_deferred_qkv_matches_epilogue_round(dev, T, bs, lora, ctx_hi):
    ops = _ops()
    H, HQ, KV, HD = 4096, 32, 8, 128
    QKV = (HQ + 2 * KV) * HD
    g = torch.Generator().manual_seed(123 + T)
    w = randn((QKV, H), 77, std=0.02)
    xs = [randn((1, H), SEED_X * 300 + i) for i in range(T)]
    table = ops.LoraTable(dev) if lora else None
    ids = None
    if lora:
        ids = []
        for i in range(T):
            A = randn((3 * 16, H), 5000 + 2 * i, std=0.02)
            Bs = [randn((d, 16), 5001 + 2 * i + 97 * j, std=0.02) for j, d in enumerate((HQ * HD, KV * HD, KV * HD))]
            ids.append(table.add(ops.pack_weight(A.to(dev)), [b.to(dev).contiguous() for b in Bs], 16, 2.0))
    ctx = torch.randint(1, ctx_hi, (T,), generator=g)
    mb = (int(ctx.max()) + 1 + bs - 1) // bs
    nb = T * mb + 3
    bt = torch.randperm(nb, generator=g)[:T * mb].to(torch.int32).reshape(T, mb)
    k0 = randn((nb, bs, KV, HD), 41)
    v0 = randn((nb, bs, KV, HD), 42)
    seql = ctx.to(torch.int32)
    pos = seql.long()
    cs = ref.cos_sin_cache(ref.rope_inv_freq(HD, 500000.0), mb * bs + 4)
    pw = ops.pack_weight(w.to(dev))
    xd = [x.to(dev) for x in xs]
    kw = dict(seg_lora=ids, table=table, blk_cols=[HQ * HD, KV * HD, KV * HD]) if lora else {}
    btd, seqd, posd, csd = bt.to(dev), seql.to(dev), pos.to(dev), cs.to(dev)
    scale = 1.0 / math.sqrt(HD)

    # epilogue path: out_mode 3 (RoPE + append), then attention rope 2
    kc_e, vc_e = k0.to(dev), v0.to(dev)
    rows_e = [torch.zeros(1, QKV, dtype=BF16, device=dev) for _ in range(T)]
    fz3 = ops.round_fusion(out_mode=3, k_cache=kc_e, v_cache=vc_e, hq=HQ, hkv=KV, block_table=btd,
                           cache_seqlens=seqd, positions=posd, cos_sin=csd)
    ops.round_ex(xd, rows_e, [1] * T, pw, None, fusion=fz3, **kw)
    out_e = [torch.zeros(1, HQ * HD, dtype=BF16, device=dev) for _ in range(T)]
    ops.paged_attention_rows([r[0] for r in rows_e], [o[0] for o in out_e], 1, HQ, KV, HD, kc_e, vc_e, btd, seqd, None, None, scale, rope=2)

    # deferred path: out_mode 4, then attention rope 3
    kc_d, vc_d = k0.to(dev), v0.to(dev)
    rows_d = [torch.zeros(1, QKV, dtype=BF16, device=dev) for _ in range(T)]
    rec = ops.QkvPartials()
    ops.round_ex(xd, rows_d, [1] * T, pw, None, fusion=ops.round_fusion(out_mode=4, defer=rec), **kw)
    out_d = [torch.zeros(1, HQ * HD, dtype=BF16, device=dev) for _ in range(T)]
    ops.paged_attention_rows([r[0] for r in rows_d], [o[0] for o in out_d], 1, HQ, KV, HD, kc_d, vc_d, btd, seqd, posd, csd, scale, rope=3,
                             qkv_partials=rec)
    torch.cuda.synchronize()

    kce, vce, kcd, vcd = kc_e.cpu(), vc_e.cpu(), kc_d.cpu(), vc_d.cpu()
    touched = torch.zeros(nb, bs, dtype=torch.bool)
    for i in range(T):
        p = int(seql[i])
        blk, off = int(bt[i, p // bs]), p % bs
        touched[blk, off] = True
        for name, a, b in (("k", kce[blk, off], kcd[blk, off]), ("v", vce[blk, off], vcd[blk, off])):
            # per head row: within two bf16 steps at the row's scale (the
            # K-slice sums differ in order; RoPE's difference of products can
            # cancel, so a one-ulp input difference is not one ulp of the output)
            d = (a.float() - b.float()).abs().amax(-1)
            lim = a.float().abs().amax(-1) / 128
            assert (d <= lim).all(), f"token {i}: appended {name} off by {d.max():.3g} (limit {lim.min():.3g})"
    assert torch.equal(kcd[~touched], k0[~touched]) and torch.equal(vcd[~touched], v0[~touched]), \
        "deferred path changed page entries other than the new keys"
    got = torch.cat([o.cpu() for o in out_d], 0)
    want_e = torch.cat([o.cpu() for o in out_e], 0)
    assert_close(got, want_e, what="attention output, deferred vs epilogue round")
    # against the oracle: the plain round's (unrotated) q, k, v through the
    # oracle's RoPE, append and attention over the original pages
    plain = [torch.zeros(1, QKV, dtype=BF16, device=dev) for _ in range(T)]
    ops.round_ex(xd, plain, [1] * T, pw, None, **kw)
    torch.cuda.synchronize()
    u = torch.cat([r.cpu() for r in plain], 0).reshape(T, 1, HQ + 2 * KV, HD)
    want, _, _ = ref.paged_attention(u[:, :, :HQ].contiguous(), u[:, :, HQ:HQ + KV].contiguous(),
                                     u[:, :, HQ + KV:].contiguous(), k0.clone(), v0.clone(), bt, seql, pos, cs, scale)
    assert_close(got.reshape(T, 1, HQ * HD), want.reshape(T, 1, HQ * HD), what="attention vs oracle")


def test_deferred_qkv_refused_where_unsupported(dev):
    ops = _ops()
    with pytest.raises(ValueError, match="QkvPartials"):
        ops.round_fusion(out_mode=4)
    rec = ops.QkvPartials()
    kc = torch.zeros(4, 16, 1, 128, dtype=BF16, device=dev)
    rows = [torch.zeros(3 * 128, dtype=BF16, device=dev)]
    out = [torch.zeros(128, dtype=BF16, device=dev)]
    bt = torch.zeros(1, 4, dtype=torch.int32, device=dev)
    sl = torch.zeros(1, dtype=torch.int32, device=dev)
    pos = torch.zeros(1, dtype=torch.int64, device=dev)
    cs = torch.zeros(64, 128, dtype=BF16, device=dev)
    with pytest.raises(ValueError, match="rope 3"):
        ops.paged_attention_rows(rows, out, 1, 1, 1, 128, kc, kc, bt, sl, pos, cs, 1.0, rope=3)
    # an empty record is not the partials of a QKV round of these sequences
    with pytest.raises(RuntimeError, match="partials"):
        ops.paged_attention_rows(rows, out, 1, 1, 1, 128, kc, kc, bt, sl, pos, cs, 1.0, rope=3, qkv_partials=rec)
