"""The prefill layer in one call (mxmoe_moe_prefill: router, blockwise mapping, M-tile
schedule and the moe_cte flow) against the operator sequence the reference model calls
(router -> build_blockwise_mapping -> moe_cte, model_mxfp4.py:1337-1433), each its own
library call.  The fused front end forms the logits with the router kernel's arithmetic
(same K quarters and MFMA sequence, quarters summed in the same order) and builds the
same mapping, so the outputs are equal bit for bit; the layer-level parity against the
oracle runs through the fused call in the other prefill tests."""

import pytest
import torch

from moe_helpers import build

pytestmark = pytest.mark.gpu


def _equal(layer, x, pm=None):
    for dt in (torch.float32, torch.bfloat16):
        a = layer.prefill(x, padding_mask=pm, output_dtype=dt)
        b = layer.prefill_ops(x, padding_mask=pm, output_dtype=dt)
        torch.cuda.synchronize()
        assert a.dtype == b.dtype == dt
        nd = int((a != b).sum())
        assert nd == 0, f"{nd} of {a.numel()} outputs differ ({dt})"


@pytest.mark.parametrize("case", [
    # (shape, E override, T, zipf, seed): ragged token counts, E not a multiple of 64
    # (one 64-expert logits tile, 16 experts per wave), E of 128 and 256 (128 experts per
    # workgroup, two expert tiles at 256) with top-8 on a narrow layer.
    ("mini", None, 300, None, 41),
    ("mini", None, 1, None, 42),
    ("mini", None, 17, None, 43),
    ("20b", None, 4096, None, 44),
    ("20b", None, 4096, 1.2, 45),
    ("20b", 40, 777, None, 46),
    ("120b", None, 4096, None, 47),
    ("wide_e", None, 1000, 1.0, 48),
])
def test_fused_prefill_equals_operator_sequence(dev, case):
    from vllm_neuron_amd import synthetic

    name, E, T, zipf, seed = case
    shape = {"mini": synthetic.MoEShape("mini", 8, 2, 256, 512),
             "20b": synthetic.GPT_OSS_20B, "120b": synthetic.GPT_OSS_120B,
             "wide_e": synthetic.MoEShape("wide-e", 256, 8, 1024, 512, swiglu_limit=None,
                                          biases=False)}[name]
    print(f"fused prefill {name} E={E} T={T} zipf={zipf}", flush=True)
    big = name == "120b"
    _, layer, _ = build(shape, seed, dev, E=E, zipf=zipf, lazy=True, pack_on_gpu=big)
    x = synthetic.tokens(seed, T, shape.H).to(dev)
    _equal(layer, x)


def test_fused_prefill_padding_mask(dev):
    from vllm_neuron_amd import synthetic

    _, layer, _ = build(synthetic.GPT_OSS_20B, 49, dev, lazy=True)
    T = 1500
    x = synthetic.tokens(49, T, 2880).to(dev)
    g = torch.Generator().manual_seed(49)
    pm = (torch.rand(T, generator=g) < 0.8).to(dev)
    _equal(layer, x, pm)
    # padded tokens contribute nothing: their rows are zero
    out = layer.prefill(x, padding_mask=pm, output_dtype=torch.float32)
    assert bool((out[~pm] == 0).all())


def test_fused_prefill_fp16_router_and_bias(dev):
    """fp16 router weights (exact split into two bf16 MFMAs, as an fp32 matmul) with an
    fp32 router bias."""
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.layer import MXFP4MoE

    shape = synthetic.MoEShape("mini", 16, 4, 512, 256)
    _, layer, lt = build(shape, 50, dev, lazy=True)
    g = torch.Generator().manual_seed(50)
    rb = (torch.randn(16, generator=g) * 0.05).to(dev)
    lay16 = MXFP4MoE(layer.w, lt.router_w.to(dev).to(torch.float16), rb, shape.K,
                     shape.swiglu_limit)
    x = synthetic.tokens(50, 333, shape.H).to(dev)
    _equal(lay16, x)


def test_fused_prefill_workspace_error(dev):
    """A workspace smaller than the query is refused with the library's error."""
    from vllm_neuron_amd import _lib, synthetic

    _, layer, _ = build(synthetic.MoEShape("mini", 8, 2, 256, 512), 51, dev, lazy=True)
    L = _lib.lib()
    w = layer.w
    T = 64
    need = L.mxmoe_moe_prefill_workspace_bytes(T, w.H, w.I, w.E, layer.top_k, 256)
    assert need > 256
    x = synthetic.tokens(51, T, w.H).to(dev)
    out = torch.empty(T, w.H, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(need - 256, dtype=torch.uint8, device=dev)
    rc = L.mxmoe_moe_prefill(
        x.data_ptr(), layer.router_w.data_ptr(), _lib.DT_BF16, None, _lib.DT_BF16,
        _lib.ROUTER_SOFTMAX, 0, 0, 0.0, _lib.DT_F32, None, w.gu_q.data_ptr(), w.gu_s.data_ptr(),
        w.dn_q.data_ptr(), w.dn_s.data_ptr(), _lib.WFMT_MXFP4, _lib.ptr(w.gu_bias),
        _lib.ptr(w.dn_bias), T, w.H, w.I, w.E, layer.top_k, 256, layer.act, layer._clamps, 0,
        out.data_ptr(), ws.data_ptr(), ws.numel(), None, _lib.stream_handle(dev))
    assert rc == -3  # MXMOE_E_WORKSPACE
    assert b"workspace" in L.mxmoe_last_error()


@pytest.mark.parametrize("E,K", [(8, 1), (16, 3), (32, 5)])
def test_fused_prefill_top_k_counts(dev, E, K):
    """Top-k counts other than 2, 4 and 8: the combine reads the first K of its 4 or 8
    per-token pair entries (the rest re-read entry 0 and are dropped) and sorts them by
    expert.  Against the operator sequence bit for bit, and against the oracle."""
    from moe_helpers import PREFILL_FP32_MEAN, check_close, routing_agreement
    from vllm_neuron_amd import synthetic

    shape = synthetic.MoEShape(f"top{K}", E, K, 256, 512)
    ref, layer, _ = build(shape, 60 + K, dev, exp=(118, 122))
    x = synthetic.tokens(60 + K, 513, shape.H)
    print(f"fused prefill top-{K} of {E}", flush=True)
    _equal(layer, x.to(dev))
    aff, ties = routing_agreement(layer, ref, x, dev)
    got = layer.prefill(x.to(dev), output_dtype=torch.float32).cpu()
    want = ref.prefill_routed(x, aff)
    check_close(got, want, ties, f"fused prefill top-{K}", mean_bound=PREFILL_FP32_MEAN)
