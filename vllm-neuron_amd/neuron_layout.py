"""Converter from vllm-neuron's Trainium MXFP4 kernel layout to this build's packed layout.

The reference prepares its MoE weights at load time into a layout tiled for its
Trainium kernels (vllm_neuron/model/gpt_oss/weight_loaders_mxfp4.py:243-885): gate/up
de-interleaved and padded to (H_pad, I_pad), fp4 pairs repacked four to a uint16,
transposed and tiled by 512-wide H and I tiles; the down projection and bias have their
hidden dim shuffled ([H] -> [H/4, 4] -> [4, H/4]).  Tensors that already went through
those loaders (one tensor-parallel rank, tp_degree = 1) can be handed to
``experts_from_neuron_layout``, which undoes each step and packs the result like a
checkpoint (``MXFP4Experts.from_split``).  The kernels work at the true H and I (no
padding), so the padded tail is dropped.

Every step is a pure permutation of bytes (torch views, permutes and slices); the
16-bit words move as int16, which every torch device can copy.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from .weights import MXFP4Experts

PMAX, Q_WIDTH, Q_HEIGHT = 128, 4, 8  # the reference's tile constants (:27-29)


def _h_tiling(H: int):
    if H % (PMAX * Q_WIDTH):
        raise ValueError(f"padded hidden size {H} must be a multiple of {PMAX * Q_WIDTH}")
    return H // (PMAX * Q_WIDTH), 512 // (Q_WIDTH * Q_HEIGHT)


def _i_tiling(I_shard: int):
    mx = Q_WIDTH * Q_HEIGHT
    if I_shard > 512:
        if I_shard % 512:
            raise ValueError(f"padded intermediate size {I_shard} must be a multiple of 512")
        return math.ceil(I_shard / 512), 512 // mx
    if I_shard % mx:
        raise ValueError(f"intermediate size {I_shard} must be a multiple of {mx}")
    return 1, I_shard // mx


def _inverse(perm):
    inv = [0] * len(perm)
    for i, p in enumerate(perm):
        inv[p] = i
    return inv


def untile_gate_up_blocks(w: torch.Tensor, H_pad: int, I_pad: int) -> torch.Tensor:
    """[E, 128, 2, H_pad/512, ...] 16-bit words -> [E, H_pad/4, 2 I_pad] (gate | up)."""
    E = w.shape[0]
    nHt, qbH = _h_tiling(H_pad)
    nIt, qbI = _i_tiling(I_pad)
    perm = (0, 2, 3, 4, 1, 5, 8, 6, 7, 9)
    y = w.reshape(E, qbH, Q_HEIGHT, 2, nHt, nIt, Q_WIDTH, qbI, Q_HEIGHT, Q_WIDTH // 4)
    return y.permute(*_inverse(perm)).reshape(E, H_pad // 4, 2 * I_pad)


def untile_gate_up_scale(s: torch.Tensor, H_pad: int, I_pad: int) -> torch.Tensor:
    """[E, 16, 2, H_pad/512, I_pad] -> [E, H_pad/32, 2 I_pad]."""
    E = s.shape[0]
    nHt, qbH = _h_tiling(H_pad)
    nIt, qbI = _i_tiling(I_pad)
    perm = (0, 2, 3, 1, 4, 7, 5, 6)
    y = s.reshape(E, qbH, 2, nHt, nIt, Q_WIDTH, qbI, Q_HEIGHT)
    return y.permute(*_inverse(perm)).reshape(E, H_pad // 32, 2 * I_pad)


def untile_gate_up_bias(b: torch.Tensor, I_pad: int) -> torch.Tensor:
    """[E, 2 I_pad] tiled -> [E, 2, I_pad] (gate, up)."""
    E = b.shape[0]
    nIt, qbI = _i_tiling(I_pad)
    perm = (0, 3, 4, 1, 2, 5)
    y = b.reshape(E, qbI, Q_HEIGHT, 2, nIt, Q_WIDTH)
    return y.permute(*_inverse(perm)).reshape(E, 2, I_pad)


def untile_down_blocks(w: torch.Tensor, H_pad: int, I_pad: int) -> torch.Tensor:
    """[E, 128, I_pad/512, H_pad] 16-bit words -> [E, I_pad/4, H_pad]."""
    E = w.shape[0]
    nIt, qbI = _i_tiling(I_pad)
    perm = (0, 2, 3, 1, 5, 4, 6)
    y = w.reshape(E, qbI, Q_HEIGHT, nIt, 4, H_pad // 4, Q_WIDTH // 4)
    return y.permute(*_inverse(perm)).reshape(E, I_pad // 4, H_pad)


def untile_down_scale(s: torch.Tensor, H_pad: int, I_pad: int) -> torch.Tensor:
    """[E, 16, I_pad/512, H_pad] -> [E, I_pad/32, H_pad]."""
    E = s.shape[0]
    nIt, qbI = _i_tiling(I_pad)
    perm = (0, 2, 1, 4, 3)
    y = s.reshape(E, qbI, nIt, 4, H_pad // 4)
    return y.permute(*_inverse(perm)).reshape(E, I_pad // 32, H_pad)


def unshuffle_hidden_dim(t: torch.Tensor, dim: int = -1) -> torch.Tensor:
    """Inverse of [H] -> [H/4, 4] -> [4, H/4] -> [H] along ``dim``."""
    if dim < 0:
        dim += t.ndim
    pre, H, post = t.shape[:dim], t.shape[dim], t.shape[dim + 1:]
    return t.reshape(*pre, 4, H // 4, *post).transpose(dim, dim + 1).reshape(*pre, H, *post)


def experts_from_neuron_layout(gate_up_blocks: torch.Tensor, gate_up_scales: torch.Tensor,
                               down_blocks: torch.Tensor, down_scales: torch.Tensor, H: int,
                               I: int, gate_up_bias: Optional[torch.Tensor] = None,
                               down_bias: Optional[torch.Tensor] = None) -> MXFP4Experts:
    """Tensors in the reference's kernel layout (one rank, padded to H_pad, I_pad) ->
    packed experts at the true sizes H, I.

    gate_up_blocks [E, 128, 2, H_pad/512, ...] uint16 (fp4 x4), gate_up_scales
    [E, 16, 2, H_pad/512, I_pad] uint8, down_blocks [E, 128, I_pad/512, H_pad] uint16,
    down_scales [E, 16, I_pad/512, H_pad] uint8, gate_up_bias [E, 2 I_pad] (tiled; the
    up half already carries the loader's hidden-activation bias), down_bias [E, H_pad]
    (hidden dim shuffled).  The padded sizes follow from the tensor shapes."""
    if gate_up_blocks.dtype not in (torch.uint16, torch.int16):
        raise TypeError("gate_up_blocks must be uint16 (four e2m1 codes each)")
    E = gate_up_blocks.shape[0]
    H_pad = gate_up_blocks.shape[3] * 512
    I_pad = gate_up_scales.shape[4]
    if H > H_pad or I > I_pad or H % 32 or I % 32:
        raise ValueError(f"H={H}, I={I} must be multiples of 32 within the padded {H_pad}, {I_pad}")
    # gate_up: untile, transpose back, bytes [E, 2 I_pad, H_pad/32, 16], split, trim
    g = untile_gate_up_blocks(gate_up_blocks.view(torch.int16), H_pad, I_pad)
    g = g.transpose(1, 2).contiguous().view(torch.uint8).reshape(E, 2 * I_pad, H_pad // 32, 16)
    gate_b, up_b = g[:, :I], g[:, I_pad:I_pad + I]
    s = untile_gate_up_scale(gate_up_scales, H_pad, I_pad).transpose(1, 2)
    gate_s, up_s = s[:, :I], s[:, I_pad:I_pad + I]
    gate_b, up_b = gate_b[:, :, :H // 32], up_b[:, :, :H // 32]
    gate_s, up_s = gate_s[:, :, :H // 32], up_s[:, :, :H // 32]
    # down: untile -> [E, I_pad/4, H_pad] uint16 -> bytes [E, H_pad, I_pad/32, 16]
    d = untile_down_blocks(down_blocks.view(torch.int16), H_pad, I_pad)
    d = d.contiguous().view(torch.uint8).reshape(E, I_pad // 4, H_pad, 2)
    d = d.transpose(1, 2).contiguous().reshape(E, H_pad, I_pad // 32, 16)[:, :H, :I // 32]
    ds = untile_down_scale(down_scales, H_pad, I_pad).transpose(1, 2)[:, :H, :I // 32]
    gub = None
    if gate_up_bias is not None:
        gub = untile_gate_up_bias(gate_up_bias, I_pad)[:, :, :I].contiguous()
    dnb = None
    if down_bias is not None:
        dnb = unshuffle_hidden_dim(down_bias, -1)[:, :H].contiguous()
    return MXFP4Experts.from_split(gate_b.contiguous(), gate_s.contiguous(), up_b.contiguous(),
                                   up_s.contiguous(), d.contiguous(), ds.contiguous(), gub, dnb)
