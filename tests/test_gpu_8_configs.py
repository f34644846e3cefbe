"""The two largest workload shapes against the oracle, on sampled tokens.

* GPT-OSS-120B-shaped layer (E=128, top-4, H=I=2880) at prefill, 4096 tokens, uniform
  routing and Zipf(1.2)-skewed routing: 382 M-tiles of 128 slots, the shape the
  prefill GEMMs are tuned for.
* Fine-grained layer (E=256, top-8, H=7168, I=2048, plain SwiGLU, no biases) with
  Zipf(1.0) routing, decode at 128 tokens and prefill at 8192 tokens.
Per-token outputs depend only on the token's own row and routing, so a sample of rows
checked against the oracle's routed forms (weights dequantized per expert on first
use) tests the whole batch's schedule.  Routing indices are compared exactly for every
token (near-ties exempted and counted).
"""

import pytest
import torch

from moe_helpers import build, check_close, decode_checked, routing_agreement

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def fine_grained(dev):
    from vllm_neuron_amd import synthetic

    _say("building the 256-expert layer (6 GB of packed weights)")
    out = build(synthetic.FINE_GRAINED, 81, dev, zipf=1.0, lazy=True, pack_on_gpu=True)
    _say("built")
    return out


@pytest.mark.timeout(600)
@pytest.mark.parametrize("zipf", [None, 1.2])
def test_prefill_gptoss120b_t4096(dev, zipf):
    from vllm_neuron_amd import synthetic

    _say(f"120B prefill T=4096 zipf={zipf}: building")
    ref, layer, _ = build(synthetic.GPT_OSS_120B, 82 if zipf is None else 83, dev, zipf=zipf,
                          lazy=True, pack_on_gpu=True)
    T = 4096
    x = synthetic.tokens(84, T, ref.H)
    aff, ties = routing_agreement(layer, ref, x, dev)
    got = layer.prefill(x.to(dev)).cpu()
    torch.cuda.synchronize()
    rows = torch.arange(3, T, T // 40)
    _say(f"oracle on {len(rows)} rows")
    want = ref.prefill_routed(x, aff, token_rows=rows)
    per_expert = (aff != 0).sum(0)
    _say(f"tokens per expert: max {int(per_expert.max())}, min {int(per_expert.min())}")
    check_close(got[rows], want, ties[rows], f"prefill 120b T=4096 zipf={zipf}")


@pytest.mark.timeout(600)
def test_decode_fine_grained_t128(dev, fine_grained):
    from vllm_neuron_amd import synthetic

    ref, layer, _ = fine_grained
    T = 128
    x = synthetic.tokens(85, T, ref.H)
    got, aff, ties = decode_checked(layer, ref, x, dev)
    rows = torch.arange(0, T, 8)
    _say(f"oracle on {len(rows)} rows")
    want = ref.decode_routed(x[rows], aff[rows])
    check_close(got[rows], want, ties[rows], "decode 256x8 T=128 zipf=1.0")


@pytest.mark.timeout(600)
def test_prefill_fine_grained_t8192(dev, fine_grained):
    from vllm_neuron_amd import synthetic

    ref, layer, _ = fine_grained
    T = 8192
    x = synthetic.tokens(86, T, ref.H)
    aff, ties = routing_agreement(layer, ref, x, dev)
    got = layer.prefill(x.to(dev)).cpu()
    torch.cuda.synchronize()
    rows = torch.arange(5, T, T // 24)
    _say(f"oracle on {len(rows)} rows")
    want = ref.prefill_routed(x, aff, token_rows=rows)
    check_close(got[rows], want, ties[rows], "prefill 256x8 T=8192 zipf=1.0")
