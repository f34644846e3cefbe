"""Deterministic synthetic inputs for the MXFP4 MoE workloads.

Bits come from numpy's PCG64 raw 64-bit words (an algorithm fixed across numpy
versions) with this module's own transforms, so identical seeds give identical
tensors on every machine of this image:
  * random bytes: the raw words viewed as little-endian bytes (uniform nibble codes);
  * integers in [lo, hi]: ((w >> 32) * (hi - lo + 1)) >> 32, then + lo;
  * normals: Box-Muller in float64 from 53-bit uniforms, rounded to bf16.

Workload shapes (per MoE layer):
  gpt-oss-20b   E=32,  top-4, H=I=2880, clamped SwiGLU (alpha 1.702, limit 7), biases
  gpt-oss-120b  E=128, top-4, H=I=2880, same expert block
  fine-grained  E=256, top-8, H=7168, I=2048, plain SwiGLU, no biases
MXFP4 weights: codes uniform over 0..15, E8M0 exponents uniform over [120, 130];
biases and router weights N(0, 0.02); tokens N(0, 1).  Routing skew adds the log-prior
-s * ln(1 + pi(e)) of a Zipf(s) law over a seeded permutation pi of expert ids to the
router logits (as a router bias).
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch


def _raw(seed: int, n: int) -> np.ndarray:
    return np.random.Generator(np.random.PCG64(seed)).bit_generator.random_raw(n)


def rand_bytes(seed: int, n: int) -> np.ndarray:
    return _raw(seed, (n + 7) // 8).view(np.uint8)[:n].copy()


def rand_ints(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    w = _raw(seed, n) >> np.uint64(32)
    return (lo + ((w * np.uint64(hi - lo + 1)) >> np.uint64(32))).astype(np.int64)


def rand_normal(seed: int, n: int) -> np.ndarray:
    m = (n + 1) // 2
    w = _raw(seed, 2 * m)
    u1 = ((w[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53  # (0, 1]
    u2 = (w[1::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53           # [0, 1)
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.concatenate([r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)])
    return z[:n]


def normal_bf16(seed: int, shape, std: float = 1.0) -> torch.Tensor:
    n = int(np.prod(shape))
    z = (rand_normal(seed, n) * std).astype(np.float32)
    return torch.from_numpy(z).reshape(shape).to(torch.bfloat16)


def mxfp4_tensor(seed: int, rows: int, K: int, exp_lo: int = 120, exp_hi: int = 130, lead=()):
    """OCP MXFP4 [..., rows, K/32, 16] blocks + [..., rows, K/32] scales."""
    G = K // 32
    nb = int(np.prod(lead, dtype=np.int64)) * rows * G * 16
    blocks = torch.from_numpy(rand_bytes(seed, nb)).reshape(*lead, rows, G, 16)
    sc = rand_ints(seed + 7919, nb // 16, exp_lo, exp_hi).astype(np.uint8)
    scales = torch.from_numpy(sc).reshape(*lead, rows, G)
    return blocks, scales


def mxfp8_tensor(seed: int, rows: int, K: int, exp_lo: int = 117, exp_hi: int = 121, lead=()):
    """OCP MXFP8 [..., rows, K/32, 32] E4M3FN codes + [..., rows, K/32] E8M0 scales; the codes
    keep exponent fields 3..10 (magnitudes 2^-4 .. 2^3 x 1.875) with random signs and
    mantissas, so that the scales set the range."""
    G = K // 32
    n = int(np.prod(lead, dtype=np.int64)) * rows * G * 32
    raw = rand_bytes(seed, n)
    e = 3 + (raw.astype(np.int64) >> 4) % 8
    codes = ((raw & 0x80) | (e << 3) | (raw & 7)).astype(np.uint8)
    sc = rand_ints(seed + 7919, n // 32, exp_lo, exp_hi).astype(np.uint8)
    return (torch.from_numpy(codes).reshape(*lead, rows, G, 32),
            torch.from_numpy(sc).reshape(*lead, rows, G))


def zipf_bias(seed: int, E: int, s: float) -> torch.Tensor:
    perm = np.argsort(_raw(seed, E), kind="stable")
    rank = np.empty(E, dtype=np.int64)
    rank[perm] = np.arange(E)
    b = (-s * np.log1p(rank.astype(np.float64))).astype(np.float32)
    return torch.from_numpy(b).to(torch.bfloat16)


@dataclass(frozen=True)
class MoEShape:
    name: str
    E: int
    K: int
    H: int
    I: int
    swiglu_limit: Optional[float] = 7.0   # None: plain SwiGLU (SiLU, no clamps)
    biases: bool = True

    @property
    def gptoss(self) -> bool:
        return self.swiglu_limit is not None


GPT_OSS_20B = MoEShape("gpt-oss-20b", 32, 4, 2880, 2880)
GPT_OSS_120B = MoEShape("gpt-oss-120b", 128, 4, 2880, 2880)
FINE_GRAINED = MoEShape("fine-grained-256x8", 256, 8, 7168, 2048, swiglu_limit=None, biases=False)


@dataclass
class LayerTensors:
    """Checkpoint-layout tensors of one MoE layer (CPU)."""
    shape: MoEShape
    gate_up_blocks: torch.Tensor   # [E, 2I, H/32, 16], rows interleaved gate/up
    gate_up_scales: torch.Tensor   # [E, 2I, H/32]
    down_blocks: torch.Tensor      # [E, H, I/32, 16]
    down_scales: torch.Tensor      # [E, H, I/32]
    gate_up_bias: Optional[torch.Tensor]  # [E, 2I] bf16, interleaved, without the +1
    down_bias: Optional[torch.Tensor]     # [E, H] bf16
    router_w: torch.Tensor         # [E, H] bf16
    router_b: Optional[torch.Tensor]      # [E] bf16


def layer_tensors(shape: MoEShape, seed: int, zipf_s: Optional[float] = None,
                  exp_range=(120, 130), E: Optional[int] = None) -> LayerTensors:
    """Seeded layer; ``E`` overrides the expert count (smaller test layers)."""
    E = shape.E if E is None else E
    H, I = shape.H, shape.I
    gub, gus = mxfp4_tensor(seed * 100 + 1, 2 * I, H, *exp_range, lead=(E,))
    dnb, dns = mxfp4_tensor(seed * 100 + 2, H, I, *exp_range, lead=(E,))
    gbias = normal_bf16(seed * 100 + 3, (E, 2 * I), 0.02) if shape.biases else None
    dbias = normal_bf16(seed * 100 + 4, (E, H), 0.02) if shape.biases else None
    rw = normal_bf16(seed * 100 + 5, (E, H), 0.02)
    rb = zipf_bias(seed * 100 + 6, E, zipf_s) if zipf_s else None
    return LayerTensors(shape, gub, gus, dnb, dns, gbias, dbias, rw, rb)


def tokens(seed: int, T: int, H: int) -> torch.Tensor:
    return normal_bf16(seed * 100 + 50 + T % 97, (T, H), 1.0)


def sha256(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()
