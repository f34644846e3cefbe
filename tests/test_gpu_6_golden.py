"""The HIP path through the C-ABI against the committed golden fixtures."""

from pathlib import Path

import numpy as np
import pytest
import torch

from moe_helpers import MAX_REL, MEAN_REL
from test_golden import load, rel_errors, tiny_layer_tensors

pytestmark = pytest.mark.gpu


def test_dequant_kat_gpu(dev):
    from vllm_neuron_amd.functional import dequantize_mxfp4_to_bf16

    d = load("dequant_kat.npz")
    out = dequantize_mxfp4_to_bf16(torch.from_numpy(d["blocks"]).to(dev),
                                   torch.from_numpy(d["scales"]).to(dev))
    bits = out.cpu().view(torch.int16).numpy().astype(np.uint16).reshape(256, 32)
    assert np.array_equal(bits, d["bf16_bits"])


def test_blockwise_cases_gpu(dev):
    from vllm_neuron_amd.functional import build_blockwise_mapping

    d = load("blockwise.npz")
    for i in range(5):
        T, E, K, B = (int(v) for v in d[f"c{i}_shape"])
        aff = torch.from_numpy(d[f"c{i}_aff"]).to(dev)
        am, tp, b2e, cond = build_blockwise_mapping(aff, E, K, B)
        assert np.array_equal(am.view(-1).cpu().numpy(), d[f"c{i}_aff_masked"]), i
        assert np.array_equal(tp.cpu().numpy(), d[f"c{i}_tp2id"]), i
        assert np.array_equal(b2e.cpu().numpy(), d[f"c{i}_b2e"]), i
        assert np.array_equal(cond.cpu().numpy(), d[f"c{i}_conditions"]), i


def test_router_case_gpu(dev):
    from vllm_neuron_amd import functional as NF

    d = load("router.npz")
    T, E, H, K = (int(v) for v in d["shape"])
    x = torch.from_numpy(d["x_bits"]).view(torch.bfloat16).to(dev)
    w = torch.from_numpy(d["w_bits"]).view(torch.bfloat16).to(dev)
    aff, logits = NF.router(x, w.T, K, return_logits=True)
    assert torch.allclose(logits.cpu(), torch.from_numpy(d["logits"]), rtol=1e-5, atol=1e-5)
    ids = torch.from_numpy(d["topk_ids"])
    got = torch.topk(aff.cpu(), K, 1).indices
    assert torch.equal(torch.sort(got, 1).values, torch.sort(ids, 1).values)
    assert torch.allclose(aff.cpu().gather(1, ids), torch.from_numpy(d["topk_vals"]),
                          rtol=1e-5, atol=1e-6)


def test_tiny_layer_gpu(dev):
    from vllm_neuron_amd.layer import MXFP4MoE
    from vllm_neuron_amd.weights import MXFP4Experts

    d = load("tiny_layer.npz")
    lt, x = tiny_layer_tensors(d)
    w = MXFP4Experts.from_checkpoint(lt.gate_up_blocks, lt.gate_up_scales, lt.down_blocks,
                                     lt.down_scales, lt.gate_up_bias, lt.down_bias).to(dev)
    layer = MXFP4MoE(w, lt.router_w.to(dev), None, 2, 7.0)
    dec = layer.decode(x.to(dev)).cpu()
    mx, mean = rel_errors(dec, torch.from_numpy(d["decode_bits"]).view(torch.bfloat16))
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)
    pre = layer.prefill(x.to(dev), output_dtype=torch.float32).cpu()
    mx, mean = rel_errors(pre, torch.from_numpy(d["prefill_f32"]))
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)
