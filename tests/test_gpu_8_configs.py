"""The two largest workload shapes against the oracle.

* GPT-OSS-120B-shaped layer (E=128, top-4, H=I=2880) at prefill, 4096 tokens, uniform
  routing and Zipf(1.2)-skewed routing: 382 M-tiles of 128 slots, the shape the
  prefill GEMMs are tuned for.  Every token row is checked, with fp32 output (the
  reference flow's own result type) against a regression bound at the achieved level,
  and with bf16 output (the layer's default) against the tolerance.
* Fine-grained layer (E=256, top-8, H=7168, I=2048, plain SwiGLU, no biases) with
  Zipf(1.0) routing: decode at 128 tokens on every row; prefill at 8192 tokens on the
  rows that reach every M-tile of every expert (first and last token of each expert and
  both sides of every 128-slot tile boundary) plus random rows.
The oracle's routed forms dequantize each expert on first use.  Routing indices are
compared exactly for every token (near-ties exempted and counted).
"""

import pytest
import torch

from moe_helpers import (BF16_OUT, PREFILL_FP32_MEAN, PREFILL_FP32_MEAN_PLAIN, build,
                         check_close, decode_checked, routing_agreement, stratified_rows)

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
    xd = x.to(dev)
    got32 = layer.prefill(xd, output_dtype=torch.float32).cpu()
    got16 = layer.prefill(xd).cpu()
    torch.cuda.synchronize()
    _say("oracle on all rows")
    want = ref.prefill_routed(x, aff)
    per_expert = (aff != 0).sum(0)
    _say(f"tokens per expert: max {int(per_expert.max())}, min {int(per_expert.min())}")
    check_close(got32, want, ties, f"prefill 120b T=4096 zipf={zipf} fp32",
                mean_bound=PREFILL_FP32_MEAN)
    check_close(got16, want.to(torch.bfloat16), ties, f"prefill 120b T=4096 zipf={zipf} bf16",
                ulp=BF16_OUT)


@pytest.mark.timeout(600)
def test_decode_fine_grained_t128(dev, fine_grained):
    from vllm_neuron_amd import synthetic

    ref, layer, _ = fine_grained
    T = 128
    x = synthetic.tokens(85, T, ref.H)
    got, aff, ties = decode_checked(layer, ref, x, dev)
    want = ref.decode_routed(x, aff)
    check_close(got, want, ties, "decode 256x8 T=128 zipf=1.0", ulp=BF16_OUT)


@pytest.mark.timeout(600)
def test_prefill_fine_grained_t8192(dev, fine_grained):
    from vllm_neuron_amd import synthetic

    ref, layer, _ = fine_grained
    T = 8192
    x = synthetic.tokens(86, T, ref.H)
    aff, ties = routing_agreement(layer, ref, x, dev)
    got = layer.prefill(x.to(dev), output_dtype=torch.float32).cpu()
    torch.cuda.synchronize()
    rows = stratified_rows(aff, extra=256, seed=86)
    _say(f"oracle on {len(rows)} rows (every M-tile of every expert)")
    want = ref.prefill_routed(x, aff, token_rows=rows)
    check_close(got[rows], want, ties[rows], "prefill 256x8 T=8192 zipf=1.0 fp32",
                mean_bound=PREFILL_FP32_MEAN_PLAIN)
