"""Oracle: MXFP8 (OCP E4M3FN codes + E8M0 block scales) -> bf16.

Test infrastructure only (see ``oracle/__init__.py``).

The reference lists MXFP8 as a weight format of moe_cte's block-sharded MX kernel
(vllm_neuron/functional/moe/moe_cte.py:49, :136-138, :206; the uint32 -> float8_e4m3fn_x4
reinterpretation of moe_block_tkg_wrapper.py:71-78) but holds no CPU flow for it (MX
tensors raise on the CPU path, moe_cte.py:584-615), so the element value is the OCP
Microscaling (MX) v1.0 one: E4M3FN(code) x 2^(scale - 127), with E8M0 scale 255 = NaN.
It is restated the way the reference's MXFP4 loader dequantizes
(vllm_neuron/model/gpt_oss/weight_loaders_bf16.py:264-316): decode into float32,
``torch.ldexp`` by the scale exponent, one rounding to bf16.

Pinned by tests/test_oracle_mxfp8.py: every (scale, code) pair, 256 x 256, against an
E4M3 decode from the bit fields (sign | 4-bit exponent, bias 7 | 3-bit mantissa,
exponent 0 subnormal, codes 0x7F / 0xFF NaN, no infinities) computed in float64 and
rounded once to float32 and once to bf16; element order (code i of a block is element i).
"""

from __future__ import annotations

import torch


def dequantize_mxfp8_to_bf16(codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """codes [..., G, 32] uint8 (E4M3FN, element i of the block at byte i) and scales
    [..., G] uint8 (E8M0, bias 127) -> bf16 [..., 32 G]."""
    v = codes.contiguous().view(torch.float8_e4m3fn).to(torch.float32)
    exp = (scales.to(torch.int32) - 127).unsqueeze(-1)
    out = torch.ldexp(v, exp.to(torch.float32))
    out = torch.where((scales == 255).unsqueeze(-1), torch.full_like(out, float("nan")), out)
    return out.to(torch.bfloat16).flatten(-2)


def mxfp8_linear(x: torch.Tensor, codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """y = x @ W^T with W = dequantize_mxfp8_to_bf16(codes, scales) [N, K]: fp32 products of
    the bf16 operands summed in fp32, rounded once to bf16."""
    w = dequantize_mxfp8_to_bf16(codes, scales).float()
    return (x.float() @ w.t()).to(torch.bfloat16)
