"""MXFP4 dequant (bit-exact) and the weight-only linear (single MXFP4 linear workload:
W [5760 x 2880], x [128 x 2880]) against the oracle."""

import numpy as np
import pytest
import torch

from oracle import mxfp4 as om

pytestmark = pytest.mark.gpu


def test_dequant_every_scale_and_code_bit_exact(dev):
    from vllm_neuron_amd.functional import dequantize_mxfp4_to_bf16

    codes = np.arange(32) % 16
    byte = (codes[0::2] | (codes[1::2] << 4)).astype(np.uint8)
    blocks = torch.from_numpy(np.tile(byte, (256, 1))).reshape(256, 1, 16)
    scales = torch.arange(256, dtype=torch.int32).to(torch.uint8).reshape(256, 1)
    want = om.dequantize_mxfp4_to_bf16(blocks, scales).view(torch.int16)
    got = dequantize_mxfp4_to_bf16(blocks.to(dev), scales.to(dev)).cpu().view(torch.int16)
    assert torch.equal(got, want)


@pytest.mark.parametrize("rows,K", [(5760, 2880), (7, 32), (3, 2048)])
def test_dequant_random_bit_exact(dev, rows, K):
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.functional import dequantize_mxfp4_to_bf16

    blocks, scales = synthetic.mxfp4_tensor(rows + K, rows, K, 0, 255)
    want = om.dequantize_mxfp4_to_bf16(blocks, scales).view(torch.int16)
    got = dequantize_mxfp4_to_bf16(blocks.to(dev), scales.to(dev)).cpu().view(torch.int16)
    assert torch.equal(got, want)


@pytest.mark.parametrize("M,N,K", [(128, 5760, 2880), (1, 16, 32), (37, 48, 96), (300, 64, 2048)])
def test_linear(dev, M, N, K):
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.functional import mxfp4_linear
    from vllm_neuron_amd.weights import pack_mxfp4

    blocks, scales = synthetic.mxfp4_tensor(11 + N, N, K)
    x = synthetic.normal_bf16(12 + M, (M, K))
    want = om.mxfp4_linear(x, blocks, scales).float()
    wq, ws = pack_mxfp4(blocks, scales)
    got = mxfp4_linear(x.to(dev), wq.to(dev), ws.to(dev)).float().cpu()
    d = (got - want).abs()
    # Same exact bf16 products summed in fp32 in two orders: each sum is within
    # K * 2^-24 * sum|x||w| of the exact value (recursive summation bound), then one
    # bf16 rounding each (one ulp apart at most, e.g. on a rounding tie).
    w_abs = om.dequantize_mxfp4_to_bf16(blocks, scales).float().abs()
    acc_bound = 2 * K * 2.0 ** -24 * (x.float().abs() @ w_abs.T)
    ulp = torch.maximum(want.abs(), got.abs()) * 2.0 ** -7
    assert torch.all(d <= ulp + acc_bound + 1e-30), d.max()
    frac_exact = (d == 0).float().mean().item()
    print(f"linear {M}x{N}x{K}: bit-identical fraction {frac_exact:.5f}")
    assert frac_exact > 0.99
    assert (d.mean() / want.abs().mean()).item() < 1e-5


@pytest.mark.parametrize("M,N,K", [(128, 5760, 2880), (1, 16, 32), (37, 48, 96),
                                   (256, 320, 4128), (17, 4096, 2048)])
def test_linear_few_rows_equals_tiled(dev, M, N, K):
    """x of at most 256 rows takes the row-group kernel (one wave per 16 rows of W, K in
    slabs through LDS); its output equals the tiled GEMM's bit for bit.  The tiled GEMM's
    rows come from the same x padded to 257 rows (rows are independent)."""
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.functional import mxfp4_linear
    from vllm_neuron_amd.weights import pack_mxfp4

    blocks, scales = synthetic.mxfp4_tensor(31 + N, N, K)
    x = synthetic.normal_bf16(32 + M, (M, K))
    wq, ws = pack_mxfp4(blocks, scales)
    wq, ws = wq.to(dev), ws.to(dev)
    got = mxfp4_linear(x.to(dev), wq, ws).cpu()
    xb = torch.zeros(257, K, dtype=torch.bfloat16)
    xb[:M] = x
    tiled = mxfp4_linear(xb.to(dev), wq, ws).cpu()[:M]
    assert torch.equal(got.view(torch.int16), tiled.view(torch.int16))


@pytest.mark.parametrize("M,N,K", [(1, 16, 32), (37, 48, 96), (64, 80, 416), (300, 64, 2048),
                                   (128, 5760, 2880)])
def test_linear_mxfp8(dev, M, N, K):
    """The GEMM kernel on MXFP8 weights (two row groups per wave, 32 B per lane and chunk,
    partial last chunks and N-tiles) against x @ W^T with the oracle's MX dequantization."""
    from oracle import mxfp8 as o8
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.functional import mxfp8_linear
    from vllm_neuron_amd.weights import pack_mxfp8

    codes, scales = synthetic.mxfp8_tensor(21 + N, N, K)
    x = synthetic.normal_bf16(22 + M, (M, K))
    want = o8.mxfp8_linear(x, codes, scales).float()
    wq, ws = pack_mxfp8(codes, scales)
    got = mxfp8_linear(x.to(dev), wq.to(dev), ws.to(dev)).float().cpu()
    d = (got - want).abs()
    w_abs = o8.dequantize_mxfp8_to_bf16(codes, scales).float().abs()
    acc_bound = 2 * K * 2.0 ** -24 * (x.float().abs() @ w_abs.T)
    ulp = torch.maximum(want.abs(), got.abs()) * 2.0 ** -7
    assert torch.all(d <= ulp + acc_bound + 1e-30), d.max()
    frac_exact = (d == 0).float().mean().item()
    print(f"mxfp8 linear {M}x{N}x{K}: bit-identical fraction {frac_exact:.5f}")
    assert frac_exact > 0.99
