"""Restatement of the reference's load-time MXFP4 transform into its Trainium kernel
layout, for one tensor-parallel rank (TEST INFRASTRUCTURE: what the tests check the
product's converter vllm_neuron_amd.neuron_layout, which inverts it, against).

Follows vllm_neuron/model/gpt_oss/weight_loaders_mxfp4.py:
  gate_up blocks  mxfp4_gate_up_blocks_loader :243-311, _pack_fp4_x4_uint16 :567-587,
                  _tile_gate_up_blocks :590-656
  gate_up scales  mxfp4_gate_up_scale_loader :314-357, _tile_gate_up_scale :659-711
  gate_up bias    mxfp4_gate_up_bias_loader :360-406, _tile_gate_up_bias :714-748
  down blocks     mxfp4_down_weight_loader :409-453, _tile_down_blocks :751-782
  down scales     mxfp4_down_scale_loader :456-489, _tile_down_scale :785-811
  down bias       mxfp4_down_bias_loader :492-528, _shuffle_hidden_dim :532-564
  tiling counts   _get_h_tiling_shard_i :814-831, _get_i_tiling_shard_i :834-885
with the sharding/padding helpers of vllm_neuron/utils/weight_loader.py
(get_shard :747-844, get_shard_deinterleaved :847-892, pad_to_shape :895-917) taken at
tp_degree = 1: the whole checkpoint is one shard, padded at the end of each dim to the
kernel shape (H_pad, I_pad).

Pinned by tests/test_neuron_layout.py: the reference's docstring examples
(_pack_fp4_x4_uint16 byte order :575-576, _get_i_tiling_shard_i :856-860,
get_shard_deinterleaved :869-874) and an independent element-by-element index
formula for every tiled tensor.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

PMAX, Q_WIDTH, Q_HEIGHT = 128, 4, 8  # weight_loaders_mxfp4.py:27-29


def pad_to_shape(t: torch.Tensor, shape) -> torch.Tensor:
    if tuple(t.shape) == tuple(shape):
        return t
    pad = []
    for actual, target in zip(reversed(t.shape), reversed(shape)):
        pad.extend([0, target - actual])
    return F.pad(t, pad)


def deinterleave(t: torch.Tensor, dim: int = 1):
    """get_shard_deinterleaved at one shard: even rows gate, odd rows up."""
    n = t.shape[dim]
    gate = t.narrow(dim, 0, n).index_select(dim, torch.arange(0, n, 2))
    up = t.narrow(dim, 0, n).index_select(dim, torch.arange(1, n, 2))
    return gate, up


def h_tiling(H: int):
    return H // (PMAX * Q_WIDTH), 512 // (Q_WIDTH * Q_HEIGHT)


def i_tiling(I_shard: int):
    mx = Q_WIDTH * Q_HEIGHT
    if I_shard > 512:
        assert I_shard % 512 == 0
        return math.ceil(I_shard / 512), 512 // mx
    assert I_shard % mx == 0
    return 1, I_shard // mx


def pack_fp4_x4_uint16(x: torch.Tensor) -> torch.Tensor:
    assert x.dtype == torch.uint8
    return x.view(torch.uint16)


def tile_gate_up_blocks(w: torch.Tensor) -> torch.Tensor:
    E, H4, I2 = w.shape
    nHt, qbH = h_tiling(H4 * 4)
    nIt, qbI = i_tiling(I2 // 2)
    w = w.reshape(E, nHt, qbH, Q_HEIGHT, 2, nIt, qbI, Q_HEIGHT, Q_WIDTH, Q_WIDTH // 4)
    w = w.permute(0, 2, 3, 4, 1, 5, 8, 6, 7, 9)
    return w.reshape(E, qbH * Q_HEIGHT, 2, nHt, -1)


def tile_gate_up_scale(s: torch.Tensor) -> torch.Tensor:
    E, H32, I2 = s.shape
    nHt, qbH = h_tiling(H32 * 32)
    nIt, qbI = i_tiling(I2 // 2)
    s = s.reshape(E, nHt, qbH, 2, nIt, qbI, Q_HEIGHT, Q_WIDTH)
    s = s.permute(0, 2, 3, 1, 4, 7, 5, 6)
    return s.reshape(E, qbH, 2, nHt, -1)


def tile_gate_up_bias(b: torch.Tensor) -> torch.Tensor:
    E, I2 = b.shape
    nIt, qbI = i_tiling(I2 // 2)
    b = b.reshape(E, 2, nIt, qbI, Q_HEIGHT, Q_WIDTH).permute(0, 3, 4, 1, 2, 5)
    return b.reshape(E, -1)


def tile_down_blocks(w: torch.Tensor) -> torch.Tensor:
    E, I4, H = w.shape
    nIt, qbI = i_tiling(I4 * 4)
    w = w.reshape(E, nIt, qbI, Q_HEIGHT, H // 4, 4, Q_WIDTH // 4)
    w = w.permute(0, 2, 3, 1, 5, 4, 6)
    return w.reshape(E, qbI * Q_HEIGHT, nIt, H * (Q_WIDTH // 4))


def tile_down_scale(s: torch.Tensor) -> torch.Tensor:
    E, I32, H = s.shape
    nIt, qbI = i_tiling(I32 * 32)
    s = s.reshape(E, nIt, qbI, H // 4, 4).permute(0, 2, 1, 4, 3)
    return s.reshape(E, qbI, nIt, H)


def shuffle_hidden_dim(t: torch.Tensor, dim: int) -> torch.Tensor:
    if dim < 0:
        dim += t.ndim
    pre, H, post = t.shape[:dim], t.shape[dim], t.shape[dim + 1:]
    assert H % 4 == 0
    return t.view(*pre, H // 4, 4, *post).transpose(dim, dim + 1).reshape(*pre, H, *post)


def gate_up_blocks(ckpt: torch.Tensor, H_pad: int, I_pad: int) -> torch.Tensor:
    """checkpoint [E, 2I, H/32, 16] -> kernel [E, 128, 2, H_pad/512, ...] uint16."""
    E = ckpt.shape[0]
    g, u = deinterleave(ckpt)
    shape = (E, I_pad, H_pad // 32, 16)
    b = torch.cat([pad_to_shape(g, shape), pad_to_shape(u, shape)], 1)
    b = b.contiguous().view(E, 2 * I_pad, -1)
    b = pack_fp4_x4_uint16(b).transpose(1, 2)
    return tile_gate_up_blocks(b).contiguous()


def gate_up_scales(ckpt: torch.Tensor, H_pad: int, I_pad: int) -> torch.Tensor:
    """checkpoint [E, 2I, H/32] -> kernel [E, 16, 2, H_pad/512, I_pad] uint8."""
    E = ckpt.shape[0]
    g, u = deinterleave(ckpt)
    shape = (E, I_pad, H_pad // 32)
    s = torch.cat([pad_to_shape(g, shape), pad_to_shape(u, shape)], 1).transpose(1, 2)
    return tile_gate_up_scale(s).contiguous()


def gate_up_bias(ckpt: torch.Tensor, I_pad: int, hidden_act_bias: float = 1.0) -> torch.Tensor:
    """checkpoint [E, 2I] (interleaved) -> kernel [E, 2 I_pad]; hidden_act_bias is added
    to the up half in place (bf16 storage, as the reference does)."""
    E = ckpt.shape[0]
    g, u = deinterleave(ckpt)
    actual = u.shape[1]
    g = pad_to_shape(g, (E, I_pad)).clone()
    u = pad_to_shape(u, (E, I_pad)).clone()
    if hidden_act_bias != 0.0:
        u[:, :actual].add_(torch.tensor([hidden_act_bias], dtype=torch.float32))
    return tile_gate_up_bias(torch.cat([g, u], 1)).contiguous()


def down_blocks(ckpt: torch.Tensor, H_pad: int, I_pad: int) -> torch.Tensor:
    """checkpoint [E, H, I/32, 16] -> kernel [E, 128, I_pad/512, ...] uint16."""
    E = ckpt.shape[0]
    b = pad_to_shape(ckpt, (E, H_pad, I_pad // 32, 16))
    b = b.contiguous().view(E, H_pad, -1, 2).transpose(1, 2).contiguous()
    b = pack_fp4_x4_uint16(b).view(E, -1, H_pad)
    return tile_down_blocks(b).contiguous()


def down_scales(ckpt: torch.Tensor, H_pad: int, I_pad: int) -> torch.Tensor:
    """checkpoint [E, H, I/32] -> kernel [E, 16, I_pad/512, H_pad] uint8."""
    E = ckpt.shape[0]
    s = pad_to_shape(ckpt, (E, H_pad, I_pad // 32)).transpose(1, 2)
    return tile_down_scale(s).contiguous()


def down_bias(ckpt: torch.Tensor, H_pad: int) -> torch.Tensor:
    """checkpoint [E, H] -> kernel [E, H_pad], H shuffled."""
    return shuffle_hidden_dim(pad_to_shape(ckpt, (ckpt.shape[0], H_pad)), -1).contiguous()
