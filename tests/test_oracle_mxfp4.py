"""Pins of oracle.mxfp4 (dequant + loaders) and of the product's packing transform."""

import math
import struct

import numpy as np
import pytest
import torch

from oracle import mxfp4 as om


def e2m1_value(code: int) -> float:
    """e2m1 by definition: sign bit, 2-bit exponent (bias 1), 1-bit mantissa, exp 0 subnormal."""
    s = -1.0 if code & 8 else 1.0
    e = (code >> 1) & 3
    m = code & 1
    if e == 0:
        return s * (m * 0.5)
    return s * (2.0 ** (e - 1)) * (1.0 + m * 0.5)


def f32_bits_rne_to_bf16(x: float) -> int:
    """float64 -> float32 (IEEE RNE, overflow to inf) -> bf16 (RNE); NaN -> 0xFFFF."""
    f = np.float32(x) if abs(x) < 3.5e38 or math.isnan(x) or math.isinf(x) else np.float32(
        math.copysign(math.inf, x))
    if np.isnan(f):
        return 0xFFFF
    u = struct.unpack("<I", struct.pack("<f", float(f)))[0]
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF
    return u >> 16


def closed_form_bits(code: int, scale: int) -> int:
    """The reference computes float(v) * float(2**(s-127)) in float32 (torch.ldexp
    into a bf16 buffer): 2**128 is +inf in float32, so scale 255 gives +-inf, or NaN
    for a zero code; otherwise the float64 product is exact and rounds once."""
    v = e2m1_value(code)
    if scale == 255:
        return 0xFFFF if v == 0 else (0xFF80 if code & 8 else 0x7F80)
    r = math.ldexp(v, scale - 127)
    if v == 0:
        return 0x8000 if code & 8 else 0
    if abs(r) >= 2.0 ** 128:
        return 0xFF80 if r < 0 else 0x7F80
    return f32_bits_rne_to_bf16(r)


def test_fp4_table_matches_e2m1_definition():
    for c in range(16):
        assert om.FP4_VALUES[c] == e2m1_value(c)
        assert math.copysign(1.0, om.FP4_VALUES[c]) == math.copysign(1.0, e2m1_value(c) or
                                                                      (-0.0 if c & 8 else 0.0))


def test_dequant_every_scale_and_code():
    # one block per scale value, codes 0..15 twice (low/high nibble each)
    codes = np.arange(32) % 16
    byte = (codes[0::2] | (codes[1::2] << 4)).astype(np.uint8)
    blocks = torch.from_numpy(np.tile(byte, (256, 1))).reshape(256, 1, 16)
    scales = torch.arange(256, dtype=torch.int32).to(torch.uint8).reshape(256, 1)
    out = om.dequantize_mxfp4_to_bf16(blocks, scales).view(torch.int16).numpy().astype(np.uint16)
    for s in range(256):
        for k in range(32):
            assert out[s, k] == closed_form_bits(int(codes[k]), s), (s, k)


def test_nibble_order_low_first():
    blocks = torch.zeros(1, 1, 16, dtype=torch.uint8)
    blocks[0, 0, 0] = 0x72  # low nibble 2 (1.0) -> element 0, high nibble 7 (6.0) -> element 1
    out = om.dequantize_mxfp4_to_bf16(blocks, torch.tensor([[127]], dtype=torch.uint8))
    assert out[0, 0].item() == 1.0 and out[0, 1].item() == 6.0
    assert torch.all(out[0, 2:] == 0)


def test_gate_up_deinterleave_and_bias():
    # rows [g0, u0, g1, u1] with constant codes per row
    E, I, H = 1, 2, 32
    codes = [2, 4, 6, 7]  # 1.0, 2.0, 4.0, 6.0
    blocks = torch.zeros(E, 2 * I, H // 32, 16, dtype=torch.uint8)
    for r, c in enumerate(codes):
        blocks[0, r] = c | (c << 4)
    scales = torch.full((E, 2 * I, H // 32), 127, dtype=torch.uint8)
    gu = om.gate_up_from_checkpoint(blocks, scales)  # [E, H, 2I] = [gate | up]
    assert gu.shape == (1, H, 2 * I)
    assert gu[0, 0].tolist() == [1.0, 4.0, 2.0, 6.0]  # gate0, gate1, up0, up1
    b = torch.tensor([[0.5, 0.25, -1.0, 2.0]], dtype=torch.bfloat16)
    assert om.gate_up_bias_from_checkpoint(b).tolist() == [[0.5, -1.0, 1.25, 3.0]]


def test_pack_unpack_roundtrip_and_layout():
    import pkgload
    pkgload.load()
    from vllm_neuron_amd.weights import pack_mxfp4, unpack_mxfp4

    g = torch.Generator().manual_seed(0)
    for N, K in ((16, 32), (32, 96), (48, 128), (16, 2880), (32, 320), (64, 160), (80, 2880)):
        blocks = torch.randint(0, 256, (2, N, K // 32, 16), generator=g, dtype=torch.uint8)
        scales = torch.randint(0, 256, (2, N, K // 32), generator=g, dtype=torch.uint8)
        d, s = pack_mxfp4(blocks, scales)
        assert d.shape == (2, N // 16, 8 * K) and s.shape == (2, (N + 63) // 64, 2 * K)
        b2, s2 = unpack_mxfp4(d, s)
        assert torch.equal(b2, blocks) and torch.equal(s2, scales)
        # the documented addressing, for every (row group, chunk, lane): data of lane l
        # of chunk c of row group g at g*8K + c*1024 + 16l, scale at q*2K + c*256 + 4l + r
        # (q, r = divmod(g, 4)); lanes past K in a partial last chunk hold nothing
        for g_ in range(N // 16):
            q, r = divmod(g_, 4)
            for c in range((K + 127) // 128):
                for l in range(64):
                    row, kb = 16 * g_ + l % 16, 4 * c + l // 16
                    if kb >= K // 32:
                        continue
                    o = c * 1024 + l * 16
                    assert torch.equal(d[1, g_, o:o + 16], blocks[1, row, kb])
                    assert s[1, q, c * 256 + 4 * l + r] == scales[1, row, kb]
        # padding of a partial last quad is zero
        nrg = N // 16
        if nrg % 4:
            for g_ in range(nrg, 4 * ((nrg + 3) // 4)):
                q, r = divmod(g_, 4)
                assert int(s[:, q].reshape(2, -1, 4)[..., r].sum()) == 0


def test_mxfp4_linear_oracle_is_fp32_matmul_of_dequant():
    g = torch.Generator().manual_seed(1)
    blocks = torch.randint(0, 256, (16, 2, 16), generator=g, dtype=torch.uint8)
    scales = torch.full((16, 2), 127, dtype=torch.uint8)
    x = torch.randn(3, 64, generator=g).to(torch.bfloat16)
    y = om.mxfp4_linear(x, blocks, scales)
    w = torch.tensor([[e2m1_value((int(blocks[n, k // 32, (k % 32) // 2]) >> (4 * (k % 2))) & 15)
                       for k in range(64)] for n in range(16)], dtype=torch.float64)
    want = (x.double() @ w.T).float().to(torch.bfloat16)
    # fp32 accumulation vs float64: at most one bf16 rounding step apart
    diff = (y.float() - want.float()).abs()
    ulp = want.float().abs() * 2.0 ** -7 + 1e-30
    assert torch.all(diff <= ulp)
