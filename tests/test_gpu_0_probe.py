"""Hardware behaviour the kernels rely on: MFMA operand/result layout and the CDNA4
scaled fp4 -> bf16 conversion, which agrees with the reference dequant for every scale
byte except 255 (the fused GEMMs run it; mxmoe_dequant_bf16 is bit-exact for all 256)."""

import numpy as np
import pytest
import torch

from oracle import mxfp4 as om

pytestmark = pytest.mark.gpu


def test_mfma_layout(dev):
    from vllm_neuron_amd import _lib

    g = torch.Generator().manual_seed(0)
    a = torch.randint(-8, 8, (16, 32), generator=g).to(torch.bfloat16)
    b = torch.randint(-8, 8, (16, 32), generator=g).to(torch.bfloat16)
    d = torch.empty(16, 16, dtype=torch.float32, device=dev)
    ad, bd = a.to(dev), b.to(dev)
    rc = _lib.lib().mxmoe_probe_mfma(ad.data_ptr(), bd.data_ptr(), d.data_ptr(),
                                     _lib.stream_handle(dev))
    _lib.check(rc, "probe_mfma")
    torch.cuda.synchronize()
    assert torch.equal(d.cpu(), a.float() @ b.float().T)


def test_hw_scaled_conversion_vs_reference(dev):
    from vllm_neuron_amd.functional.mxfp4 import dequantize_mxfp4_to_bf16

    codes = np.arange(32) % 16
    byte = (codes[0::2] | (codes[1::2] << 4)).astype(np.uint8)
    blocks = torch.from_numpy(np.tile(byte, (256, 1))).reshape(256, 1, 16)
    scales = torch.arange(256, dtype=torch.int32).to(torch.uint8).reshape(256, 1)
    want = om.dequantize_mxfp4_to_bf16(blocks, scales).view(torch.int16)
    got = dequantize_mxfp4_to_bf16(blocks.to(dev), scales.to(dev), _hw_probe=True)
    got = got.cpu().view(torch.int16)
    same = (got == want).all(1)
    bad = [s for s in range(256) if not bool(same[s])]
    print("hardware conversion differs from the reference at scale bytes:", bad)
    # Scale 255 (2^128) overflows fp32 in the reference (inf, and NaN for the zero codes);
    # the hardware treats it otherwise.  Every other byte, the subnormal 2^-127 of byte 0
    # and the overflowing products of bytes 253 and 254 included, agrees bit for bit.
    assert bad == [255], bad


def test_mxfp8_dequant_exact_and_hw_conversion(dev):
    """MXFP8: the library's integer dequantization and the CDNA4 scaled fp8 -> bf16
    conversion the MXFP8 GEMMs run are both bit-exact with the oracle's MX definition for
    every (scale, code) pair: scale 255 and the NaN codes give NaN, the results below
    2^-126 round to the nearest even multiple of 2^-133, the largest products overflow to
    infinity."""
    from oracle import mxfp8 as o8
    from vllm_neuron_amd.functional.mxfp4 import dequantize_mxfp8_to_bf16

    codes = torch.arange(256, dtype=torch.uint8).reshape(1, 8, 32).expand(256, 8, 32).contiguous()
    scales = torch.arange(256, dtype=torch.int32).to(torch.uint8).reshape(256, 1).expand(256, 8)
    scales = scales.contiguous()
    want = o8.dequantize_mxfp8_to_bf16(codes, scales)
    wnan = torch.isnan(want.float())
    for hw in (False, True):
        got = dequantize_mxfp8_to_bf16(codes.to(dev), scales.to(dev), _hw_probe=hw).cpu()
        gnan = torch.isnan(got.float())
        same = (got.view(torch.int16) == want.view(torch.int16)) | (gnan & wnan)
        bad = [s for s in range(256) if not bool(same[s].all())]
        print("hw" if hw else "exact", "dequant differs from the MX definition at scale bytes:",
              bad)
        assert bad == []
