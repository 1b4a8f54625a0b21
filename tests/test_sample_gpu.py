"""GPU tests of the next-token sampler (swl_sample_bf16, N1 of the path;
the reference samples in ext_aggregator.cpp:630-875 with torch on the GPU).

Greedy rows must equal torch's argmax of the same bf16 logits (first index on
ties), for vocabularies whose rows are and are not 16-byte aligned.  Sampled
rows follow the same distribution, not the same random stream: top-k keeps
the token inside the k largest logits, top-k = 1 and a tiny top-p reduce to
argmax, the seed fixes the draw, and the empirical frequencies over many rows
match softmax(logits / temperature).
"""

import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _ops():
    from swarmlora_amd import ops
    return ops


def _run(logits, do_sample, temperature=1.0, top_k=0, top_p=1.0, seed=0):
    ops = _ops()
    n = logits.shape[0]
    out = torch.full((n, 1), -1, dtype=torch.int64, device=logits.device)
    ops.sample(logits, [out[i] for i in range(n)], [do_sample] * n, [temperature] * n, [top_k] * n, [top_p] * n,
               seed=seed)
    torch.cuda.synchronize()
    return out[:, 0].cpu()


@pytest.mark.parametrize("vocab", [128256, 1001, 7, 8])
def test_greedy_is_first_argmax(dev, vocab):
    g = torch.Generator().manual_seed(vocab)
    n = 28
    lg = torch.randn(n, vocab, generator=g).to(torch.bfloat16)
    # plant ties of the row maximum at two places (the earlier one wins)
    for r in range(0, n, 3):
        i, j = sorted(torch.randint(0, vocab, (2,), generator=g).tolist())
        lg[r, i] = lg[r, j] = 40.0
    got = _run(lg.to(dev), False)
    assert torch.equal(got, lg.float().argmax(1))


def test_top_k_one_and_tiny_top_p_are_argmax(dev):
    g = torch.Generator().manual_seed(1)
    lg = torch.randn(16, 5000, generator=g).to(torch.bfloat16)
    want = lg.float().argmax(1)
    assert torch.equal(_run(lg.to(dev), True, temperature=0.8, top_k=1, seed=3), want)
    assert torch.equal(_run(lg.to(dev), True, temperature=0.8, top_p=1e-6, seed=3), want)


def test_top_k_keeps_the_k_largest_and_seed_fixes_the_draw(dev):
    g = torch.Generator().manual_seed(2)
    n, vocab, k = 64, 3000, 5
    lg = (torch.randn(n, vocab, generator=g) * 0.5).to(torch.bfloat16)
    d = lg.to(dev)
    a = _run(d, True, temperature=1.0, top_k=k, seed=11)
    b = _run(d, True, temperature=1.0, top_k=k, seed=11)
    assert torch.equal(a, b)
    kth = lg.float().topk(k, dim=1).values[:, -1]
    picked = lg.float().gather(1, a.view(-1, 1))[:, 0]
    assert bool((picked >= kth).all())
    c = _run(d, True, temperature=1.0, top_k=k, seed=12)
    assert not torch.equal(a, c)


def test_sampled_frequencies_follow_softmax(dev):
    """32 calls (seeds) x 128 rows of the same 4 logits: each draw is
    independent (seed and row index enter the hash), so the token counts
    follow softmax(l / T).  top_p keeps the tokens whose inclusive cumulative
    probability is at most top_p, and the most likely one
    (ext_aggregator.cpp:770-782)."""
    n, calls, T = 128, 32, 0.7
    row = torch.tensor([1.0, 0.5, -0.25, 0.0]).to(torch.bfloat16)
    lg = row.repeat(n, 1).to(dev)
    p = torch.softmax(row.float() / T, 0).double()   # [0.527, 0.258, 0.088, 0.126]

    def counts(**kw):
        got = torch.cat([_run(lg, True, temperature=T, seed=100 + c, **kw) for c in range(calls)])
        return torch.bincount(got, minlength=4).double()

    def check(c, q):
        tot = n * calls
        for i in range(4):
            sd = math.sqrt(tot * q[i] * (1 - q[i])) + 1e-9
            assert abs(c[i] - tot * q[i]) < 4.5 * sd + 1e-9, (i, c.tolist(), (tot * q).tolist())

    check(counts(), p)
    # cumulative [0.527, 0.785, 0.911, 1.0]: top_p 0.8 keeps tokens 0 and 1
    q = torch.tensor([p[0], p[1], 0.0, 0.0], dtype=torch.float64)
    check(counts(top_p=0.8), q / q.sum())
    # top_p 0.6 keeps only token 0
    assert counts(top_p=0.6)[0] == n * calls
    # top_k 3 drops token 2 (the smallest)
    q = torch.tensor([p[0], p[1], 0.0, p[3]], dtype=torch.float64)
    check(counts(top_k=3), q / q.sum())


@pytest.mark.parametrize("vocab,hidden", [(128256, 4096), (1001, 136)])
def test_embed_rows_bit_exact_with_clamped_ids(dev, vocab, hidden):
    """swl_embed_bf16 against the oracle's embed round (ext_aggregator.cpp:
    630-706): ragged slots, ids below 0 and at or past the vocabulary
    clamped to the first / last row, every output row bit-identical to the
    table row (the table holds arbitrary 16-bit patterns)."""
    from oracle import reference_path as ref
    from tests._util import bits_equal
    ops = _ops()
    g = torch.Generator().manual_seed(vocab)
    table = torch.randint(-32768, 32768, (vocab, hidden), generator=g, dtype=torch.int32).to(torch.int16)
    table = table.view(torch.bfloat16)
    edge = [0, vocab - 1, -1, vocab, -(1 << 40), (1 << 40), vocab + 7]
    rnd = torch.randint(0, vocab, (40,), generator=g).tolist()
    ids = [torch.tensor(edge[:3], dtype=torch.int64), torch.tensor(rnd[:16] + edge[3:], dtype=torch.int64),
           torch.tensor([], dtype=torch.int64), torch.tensor(rnd[16:], dtype=torch.int64)]
    td = table.to(dev)
    outs = [torch.full((max(t.numel(), 1), hidden), 7.0, dtype=torch.bfloat16, device=dev) for t in ids]
    ops.embed([t.to(dev) for t in ids], td, outs)
    torch.cuda.synchronize()
    want = ref.embed_round(ids, table)
    for i, (o, w) in enumerate(zip(outs, want)):
        assert bits_equal(o[: w.shape[0]].cpu(), w), f"slot {i}"
    # an empty slot's buffer is not written
    assert bool((outs[2] == 7.0).all())
