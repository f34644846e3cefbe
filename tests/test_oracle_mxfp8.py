"""Pins of oracle.mxfp8 (dequant) and of the product's MXFP8 packing transform."""

import math
import struct

import numpy as np
import torch

from oracle import mxfp8 as o8


def e4m3_value(code: int) -> float:
    """E4M3FN by definition: sign, 4-bit exponent (bias 7), 3-bit mantissa, exponent 0
    subnormal, S.1111.111 NaN, no infinities."""
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 15
    m = code & 7
    if e == 15 and m == 7:
        return math.nan
    if e == 0:
        return s * (m / 8.0) * 2.0 ** -6
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def bf16_bits(x: float) -> int:
    """float64 -> float32 (IEEE RNE, subnormals kept, overflow to inf) -> bf16 (RNE)."""
    if math.isnan(x):
        return 0x7FC0
    with np.errstate(over="ignore"):
        f = np.float32(x)
    u = struct.unpack("<I", struct.pack("<f", float(f)))[0]
    if (u & 0x7F800000) == 0x7F800000:
        return u >> 16
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF
    return u >> 16


def test_e4m3_table_matches_bit_fields():
    vals = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().tolist()
    for c in range(256):
        want = e4m3_value(c)
        if math.isnan(want):
            assert math.isnan(vals[c]), c
        else:
            assert vals[c] == want, (c, vals[c], want)
    assert e4m3_value(0x7E) == 448.0 and e4m3_value(0x01) == 2.0 ** -9


def test_every_scale_and_code_closed_form():
    codes = torch.arange(256, dtype=torch.uint8).reshape(1, 8, 32).expand(256, 8, 32)
    scales = torch.arange(256, dtype=torch.uint8).reshape(256, 1).expand(256, 8)
    got = o8.dequantize_mxfp8_to_bf16(codes.contiguous(), scales.contiguous()).view(torch.int16)
    got = got.to(torch.int32).numpy() & 0xFFFF  # [256 scales, 256 codes]
    bad = 0
    for s in range(256):
        for c in range(256):
            v = e4m3_value(c)
            g = int(got[s, c])
            if s == 255 or math.isnan(v):
                bad += (g & 0x7F80) != 0x7F80 or (g & 0x7F) == 0
                continue
            want = bf16_bits(v * 2.0 ** (s - 127))
            bad += g != want
    assert bad == 0


def test_element_order_and_block_scales():
    codes = torch.zeros(2, 3, 32, dtype=torch.uint8)
    codes[1, 2, 5] = 0x38  # 1.0
    scales = torch.full((2, 3), 127, dtype=torch.uint8)
    scales[1, 2] = 130
    out = o8.dequantize_mxfp8_to_bf16(codes, scales)
    assert out.shape == (2, 96)
    nz = torch.nonzero(out.float())
    assert nz.tolist() == [[1, 2 * 32 + 5]] and out[1, 69].item() == 8.0


def test_pack_unpack_mxfp8_round_trip():
    from vllm_neuron_amd.weights import pack_mxfp8, packed_scale_shape, unpack_mxfp8

    g = torch.Generator().manual_seed(5)
    for N, K in ((16, 128), (48, 96), (80, 416), (64, 2880)):
        codes = torch.randint(0, 256, (3, N, K // 32, 32), generator=g, dtype=torch.uint8)
        scales = torch.randint(0, 256, (3, N, K // 32), generator=g, dtype=torch.uint8)
        d, s = pack_mxfp8(codes, scales)
        assert d.shape == (3, N // 16, 16 * K) and s.shape == (3, *packed_scale_shape(N, K))
        c2, s2 = unpack_mxfp8(d, s)
        assert torch.equal(c2, codes) and torch.equal(s2, scales)


def test_pack_mxfp8_lane_layout():
    """Chunk c of row group g at g*16K + c*2048; half h (block values 16h..16h+15) at
    +h*1024; lane l = 16q + r holds row 16g + r, K-block 4c + q (tail chunk: halves of
    256 * blocks bytes)."""
    from vllm_neuron_amd.weights import pack_mxfp8

    N, K = 32, 192  # one full chunk and a 2-block tail
    G = K // 32
    codes = torch.zeros(N, G, 32, dtype=torch.uint8)
    for row in range(N):
        for b in range(G):
            for i in range(32):
                codes[row, b, i] = (row * 7 + b * 13 + i) % 251
    d, _ = pack_mxfp8(codes, torch.zeros(N, G, dtype=torch.uint8))
    d = d.reshape(-1)
    for g_ in range(N // 16):
        for row in range(16):
            for b in range(G):
                c, q = b // 4, b % 4
                for h in range(2):
                    if c < G // 4:
                        off = g_ * 16 * K + c * 2048 + h * 1024 + (16 * q + row) * 16
                    else:
                        tq = G % 4
                        off = g_ * 16 * K + (G // 4) * 2048 + h * 256 * tq + (16 * q + row) * 16
                    assert torch.equal(d[off:off + 16], codes[16 * g_ + row, b, 16 * h:16 * h + 16])
