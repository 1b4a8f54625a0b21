"""The benchmarked step itself: BASELINE config 4 at its full size (32
Llama-3.1-8B-shaped layers, 28 workers with rank-16 adapters, vocabulary
128256, paged KV contexts U{128..2048}), built exactly as bench.py builds it.

Two decoders from the same seeds: one runs eager steps, the other replays
the captured HIP graph.  Per step the two must agree bit for bit (logits,
sampled tokens, the residual stream), the logits must be finite, every
greedy token must be the first maximum of its row's logits, and the
sequence lengths must advance by one.  Numerical parity of the step against
the CPU oracle is tested at the same widths over two layers
(test_decode_config4_gpu.py); these properties cover the 32-layer graph the
benchmark times."""

import pytest
import torch

from tests._util import bits_equal

pytestmark = pytest.mark.gpu

W = 28


def _decoder(dev):
    from swarmlora_amd.decode import BatchedDecoder, DecodeShape, synthetic_adapter, synthetic_weights
    s = DecodeShape()
    ctx = torch.randint(128, 2049, (W,), generator=torch.Generator().manual_seed(3)).tolist()
    first = torch.randint(0, s.vocab, (W,), generator=torch.Generator().manual_seed(4)).tolist()
    weights = synthetic_weights(s, dev, seed=0)
    adapters = [synthetic_adapter(s, dev, seed=1000 + w) for w in range(W)]
    kv_gen = torch.Generator(device=dev).manual_seed(5)

    def kv_fill(li, kc, vc, bt):
        kc.copy_(torch.randn(kc.shape, generator=kv_gen, device=dev, dtype=torch.bfloat16))
        vc.copy_(torch.randn(vc.shape, generator=kv_gen, device=dev, dtype=torch.bfloat16))

    dec = BatchedDecoder(s, weights, adapters, ctx, first, dev, max_new=8, kv_fill=kv_fill)
    del weights, adapters
    return dec, ctx


def test_full_config4_step_graph_replays_equal_eager_steps(dev):
    print("building the eager decoder", flush=True)
    eager, ctx = _decoder(dev)
    print("building the graph decoder", flush=True)
    graph, _ = _decoder(dev)
    try:
        graph.step_eager()  # step 0 eager on both (sizes scratch, uploads the adapter table)
        eager.step_eager()
        graph.capture()
        for step in range(4):
            print(f"full config-4 step {step}: {'eager vs eager' if step == 0 else 'eager vs graph replay'}",
                  flush=True)
            if step > 0:
                eager.step_eager()
                graph.step()
            torch.cuda.synchronize()
            le, lg = eager.logits.cpu(), graph.logits.cpu()
            ie, ig = eager.ids.reshape(-1).cpu(), graph.ids.reshape(-1).cpu()
            assert bits_equal(lg, le), f"step {step}: logits differ"
            assert torch.equal(ig, ie), f"step {step}: tokens differ"
            assert bits_equal(graph.final_h.cpu(), eager.final_h.cpu()), f"step {step}: residual stream differs"
            assert torch.isfinite(le.float()).all(), f"step {step}: non-finite logits"
            lf = le.float()
            for w in range(W):
                assert int(ie[w]) == int(lf[w].argmax()), f"step {step} worker {w}: not the argmax"
            assert eager.seqlens.cpu().tolist() == [c + step + 1 for c in ctx]
    finally:
        eager.close()
        graph.close()
