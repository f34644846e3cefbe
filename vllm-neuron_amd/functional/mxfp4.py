"""MXFP4 / MXFP8 dequantization and weight-only linear on the MI355X kernels.

``dequantize_mxfp4_to_bf16`` is bit-exact with the reference loader's
``_dequantize_mxfp4_to_bf16`` (vllm_neuron/model/gpt_oss/weight_loaders_bf16.py:264-316),
including scale bytes 0 (subnormal results), 254 (overflow to inf) and 255 (inf,
NaN for zero codes).  ``mxfp4_linear`` is one expert projection as the reference CPU
flow computes it: dequantized weights, bf16 matmul with fp32 accumulation.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib


def dequantize_mxfp4_to_bf16(blocks: Tensor, scales: Tensor, _hw_probe: bool = False) -> Tensor:
    """blocks [..., G, 16] uint8 + scales [..., G] uint8 -> bf16 [..., 32G]."""
    dev = _lib.require_cuda(blocks, scales)
    if blocks.dtype != torch.uint8 or scales.dtype != torch.uint8:
        raise TypeError("blocks and scales must be uint8")
    if blocks.shape[-1] != 16 or tuple(scales.shape) != tuple(blocks.shape[:-1]):
        raise ValueError("expected blocks [..., G, 16] and scales [..., G]")
    G = blocks.shape[-2]
    rows = blocks.numel() // (G * 16) if G else 0
    out = torch.empty(*blocks.shape[:-2], G * 32, dtype=torch.bfloat16, device=dev)
    fn = _lib.lib().mxmoe_probe_hw_dequant if _hw_probe else _lib.lib().mxmoe_dequant_bf16
    rc = fn(blocks.contiguous().data_ptr(), scales.contiguous().data_ptr(), out.data_ptr(), rows,
            G * 32, _lib.stream_handle(dev))
    _lib.check(rc, "mxmoe_dequant_bf16")
    return out


def _mx_linear(x: Tensor, w_packed: Tensor, w_scale: Tensor, fmt: int, per_k: int) -> Tensor:
    dev = _lib.require_cuda(x, w_packed, w_scale)
    if x.dtype != torch.bfloat16:
        raise NotImplementedError("x must be bfloat16")
    M, K = x.shape
    N = w_packed.shape[0] * 16
    if w_packed.shape[1] != per_k * K or tuple(w_scale.shape) != ((N + 63) // 64, 2 * K):
        raise ValueError("packed weight shape does not match x")
    y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    rc = _lib.lib().mxmoe_linear(x.contiguous().data_ptr(), M, w_packed.contiguous().data_ptr(),
                                 w_scale.contiguous().data_ptr(), fmt, N, K, y.data_ptr(),
                                 _lib.stream_handle(dev))
    _lib.check(rc, "mxmoe_linear")
    return y


def mxfp4_linear(x: Tensor, w_packed: Tensor, w_scale: Tensor) -> Tensor:
    """x bf16 [M, K]; W packed [N/16, 8K] + [ceil(N/64), 2K] -> y bf16 [M, N]."""
    return _mx_linear(x, w_packed, w_scale, _lib.WFMT_MXFP4, 8)


def mxfp8_linear(x: Tensor, w_packed: Tensor, w_scale: Tensor) -> Tensor:
    """x bf16 [M, K]; W MXFP8 packed (weights.pack_mxfp8) [N/16, 16K] + [ceil(N/64), 2K] ->
    y bf16 [M, N]."""
    return _mx_linear(x, w_packed, w_scale, _lib.WFMT_MXFP8, 16)


def dequantize_mxfp8_to_bf16(codes: Tensor, scales: Tensor, _hw_probe: bool = False) -> Tensor:
    """codes [..., G, 32] uint8 (E4M3FN) + scales [..., G] uint8 (E8M0) -> bf16 [..., 32G]:
    E4M3FN(code) x 2^(scale - 127) rounded once to bf16, scale 255 -> NaN (the OCP MX
    definition; the reference has no CPU flow for MXFP8)."""
    dev = _lib.require_cuda(codes, scales)
    if codes.dtype != torch.uint8 or scales.dtype != torch.uint8:
        raise TypeError("codes and scales must be uint8")
    if codes.shape[-1] != 32 or tuple(scales.shape) != tuple(codes.shape[:-1]):
        raise ValueError("expected codes [..., G, 32] and scales [..., G]")
    G = codes.shape[-2]
    rows = codes.numel() // (G * 32) if G else 0
    out = torch.empty(*codes.shape[:-2], G * 32, dtype=torch.bfloat16, device=dev)
    L = _lib.lib()
    fn = L.mxmoe_probe_hw_dequant_fp8 if _hw_probe else L.mxmoe_dequant_mxfp8_bf16
    rc = fn(codes.contiguous().data_ptr(), scales.contiguous().data_ptr(), out.data_ptr(), rows,
            G * 32, _lib.stream_handle(dev))
    _lib.check(rc, "mxmoe_dequant_mxfp8_bf16")
    return out
