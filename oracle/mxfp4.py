"""Oracle: MXFP4 (OCP e2m1 nibbles + E8M0 block scales) -> bf16, and the CPU-path loaders.

Test infrastructure only (see ``oracle/__init__.py``).

Follows vllm_neuron/model/gpt_oss/weight_loaders_bf16.py:
  * ``dequantize_mxfp4_to_bf16``  <- ``_dequantize_mxfp4_to_bf16`` (:264-316)
  * ``gate_up_from_checkpoint``   <- ``expert_gate_up_weight_sharding_loader`` (:319-383), tp=1
  * ``gate_up_bias_from_checkpoint`` <- ``expert_gate_up_bias_sharding_loader`` (:386-422), tp=1
  * ``down_from_checkpoint``      <- ``expert_down_weight_sharding_loader`` (:425-488), tp=1

Pinned by (tests/test_oracle_mxfp4.py):
  * the FP4 table in the reference docstring (:281-302) checked entry by entry
    against the e2m1 definition (sign | 2-bit exponent, bias 1 | 1-bit mantissa,
    exponent 0 subnormal) computed independently with Python floats;
  * every (scale, code) pair, 256 x 16, against ``math.ldexp`` in float64 followed
    by one IEEE rounding to float32 and one to bf16 (closed form, including
    scale 0 -> 2^-127 subnormals, scale 254 overflow and scale 255 -> inf/NaN);
  * nibble order (low nibble = even element) on hand-built bytes;
  * gate/up de-interleave on a hand-built [gate0, up0, gate1, up1] example
    (vllm_neuron/utils/weight_loader.py:869-874 shows the same pattern).
"""

from __future__ import annotations

import torch

# e2m1 values indexed by the 4-bit code (weight_loaders_bf16.py:281-302).
FP4_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
              -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)


def dequantize_mxfp4_to_bf16(blocks: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """blocks [..., G, 16] uint8 (two e2m1 per byte, low nibble first) and
    scales [..., G] uint8 (E8M0, bias 127) -> bf16 [..., 32*G].

    Restates weight_loaders_bf16.py:264-316: table lookup into bf16
    (:281-302), exponent ``scale - 127`` (:304), even elements from the low
    nibble and odd from the high nibble (:312-313), then ``torch.ldexp`` into
    the bf16 buffer (:314).
    """
    lut = torch.tensor(FP4_VALUES, dtype=torch.bfloat16)
    exp = (scales.to(torch.int32) - 127).unsqueeze(-1)
    out = torch.empty(*blocks.shape[:-1], blocks.shape[-1] * 2, dtype=torch.bfloat16)
    out[..., 0::2] = lut[(blocks & 0x0F).long()]
    out[..., 1::2] = lut[(blocks >> 4).long()]
    torch.ldexp(out, exp, out=out)
    return out.flatten(-2)


def gate_up_from_checkpoint(blocks: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """Checkpoint gate_up_proj_{blocks,scales} [E, 2I, H/32, 16] / [E, 2I, H/32] with
    rows interleaved (2i = gate_i, 2i+1 = up_i) -> bf16 parameter [E, H, 2I] laid out
    as [gate | up] on the last dim.

    Restates weight_loaders_bf16.py:356-383 at one shard and no padding.
    """
    deq = dequantize_mxfp4_to_bf16(blocks, scales)  # [E, 2I, H]
    gate, up = deq[:, ::2], deq[:, 1::2]
    return torch.cat([gate, up], dim=1).transpose(1, 2).contiguous()


def gate_up_bias_from_checkpoint(bias: torch.Tensor) -> torch.Tensor:
    """Checkpoint gate_up_proj_bias [E, 2I] (interleaved) -> [E, 2I] = [gate | up + 1].

    Restates weight_loaders_bf16.py:393-422: de-interleave, then ``up + 1`` in the
    bias dtype (bf16), no padding at one shard.
    """
    gate = bias[:, ::2]
    up = bias[:, 1::2].clone()
    up = up + 1
    return torch.cat([gate, up], dim=1)


def down_from_checkpoint(blocks: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """Checkpoint down_proj_{blocks,scales} [E, H, I/32, 16] / [E, H, I/32] -> bf16
    parameter [E, I, H].

    Restates weight_loaders_bf16.py:450-488 at one shard and no padding.
    """
    deq = dequantize_mxfp4_to_bf16(blocks, scales)  # [E, H, I]
    return deq.transpose(1, 2).contiguous()


def mxfp4_linear(x: torch.Tensor, blocks: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """Weight-only MXFP4 linear: y = bf16(x @ dequant(W)^T) with fp32 accumulation.

    W is [N, K] as blocks [N, K/32, 16] + scales [N, K/32]; x is bf16 [M, K].
    The dequantized weights are exactly representable in bf16, so the fp32 matmul
    below is the same arithmetic as the reference's bf16 ``F.linear`` over
    weights dequantized at load (fp32 products of bf16 values are exact).
    """
    w = dequantize_mxfp4_to_bf16(blocks, scales).float()
    return (x.float() @ w.t()).to(torch.bfloat16)
