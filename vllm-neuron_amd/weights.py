"""Load-time weight preparation: checkpoint MXFP4 (and MXFP8) tensors -> the kernels'
packed layout.

The reference prepares its kernel-facing MXFP4 layout once at load
(vllm_neuron/model/gpt_oss/weight_loaders_mxfp4.py:243-885, a Trainium-specific
tiling); this module is the MI355X counterpart.  Input is the OCP/HF checkpoint
layout (vllm_neuron/model/gpt_oss/model_mxfp4.py:2069-2141):

  gate_up_proj_blocks [E, 2I, H/32, 16] uint8, gate_up_proj_scales [E, 2I, H/32] uint8,
  rows interleaved (row 2i = gate_i, row 2i+1 = up_i);
  down_proj_blocks [E, H, I/32, 16], down_proj_scales [E, H, I/32];
  gate_up_proj_bias [E, 2I] (interleaved), down_proj_bias [E, H].

Packed layout of one [N, K] matrix (rows grouped by 16, K in 128-element chunks):
  data  [N/16, 8K] bytes: chunk c of row group g at g*8K + c*1024; inside it the
        16 bytes of lane l are row 16g + l%16, K-block 4c + l//16 (a partial last
        chunk keeps only its lanes l < 16 * blocks_in_chunk);
  scale [ceil(N/64), 2K] bytes, row groups taken four at a time ("quads"): the E8M0
        byte of row group g = 4q + r, chunk c, lane l is at q*2K + c*256 + 4l + r, so
        one 32-bit word per lane holds the scales of a quad's four row groups (a
        partial last quad is padded with zero bytes).
Fused gate_up matrices alternate 16-row groups of gate and up rows.

Every function here is a pure layout transform (torch views/permutes) that runs on
whatever device its inputs live on.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch


def _pack_2d(blocks: torch.Tensor, scales: torch.Tensor):
    """blocks [L, N, G, 16], scales [L, N, G] -> data [L, N/16, 256G], scale [L, NQ, 64G]
    with NQ = ceil(N/64)."""
    L, N, G, _ = blocks.shape
    if N % 16:
        raise ValueError(f"row count {N} must be a multiple of 16")
    nrg, nfull, tq = N // 16, G // 4, G % 4
    nq = (nrg + 3) // 4
    b = blocks.reshape(L, nrg, 16, G, 16)
    s = scales.reshape(L, N, G)
    if nq * 64 != N:
        s = torch.cat([s, s.new_zeros(L, nq * 64 - N, G)], 1)
    s = s.reshape(L, nq, 4, 16, G)  # quad, r, row, block
    parts_d, parts_s = [], []
    if nfull:
        bf = b[:, :, :, :4 * nfull, :].reshape(L, nrg, 16, nfull, 4, 16)
        parts_d.append(bf.permute(0, 1, 3, 4, 2, 5).reshape(L, nrg, nfull * 1024))
        sf = s[..., :4 * nfull].reshape(L, nq, 4, 16, nfull, 4)  # quad, r, row, c, kq
        parts_s.append(sf.permute(0, 1, 4, 5, 3, 2).reshape(L, nq, nfull * 256))
    if tq:
        bt = b[:, :, :, 4 * nfull:, :]  # [L, rg, r, tq, byte]
        parts_d.append(bt.permute(0, 1, 3, 2, 4).reshape(L, nrg, tq * 256))
        st = s[..., 4 * nfull:]  # quad, r, row, kq
        parts_s.append(st.permute(0, 1, 4, 3, 2).reshape(L, nq, tq * 64))
    return torch.cat(parts_d, -1).contiguous(), torch.cat(parts_s, -1).contiguous()


def pack_mxfp4(blocks: torch.Tensor, scales: torch.Tensor):
    """OCP blocks [..., N, K/32, 16] + scales [..., N, K/32] -> packed (data, scale)
    with shapes [..., N/16, 8K] and [..., ceil(N/64), 2K]."""
    if blocks.dtype != torch.uint8 or scales.dtype != torch.uint8:
        raise TypeError("MXFP4 blocks and scales must be uint8")
    lead = blocks.shape[:-3]
    N, G = blocks.shape[-3], blocks.shape[-2]
    if blocks.shape[-1] != 16 or tuple(scales.shape) != tuple(blocks.shape[:-1]):
        raise ValueError("expected blocks [..., N, G, 16] and scales [..., N, G]")
    d, s = _pack_2d(blocks.reshape(-1, N, G, 16), scales.reshape(-1, N, G))
    return d.reshape(*lead, N // 16, G * 256), s.reshape(*lead, (N + 63) // 64, G * 64)


def _pack_scales(scales: torch.Tensor) -> torch.Tensor:
    """scales [L, N, G] -> the packed scale layout [L, ceil(N/64), 64G] (see the module
    docstring); shared by MXFP4 and MXFP8."""
    L, N, G = scales.shape
    nq, nfull, tq = (N // 16 + 3) // 4, G // 4, G % 4
    s = scales
    if nq * 64 != N:
        s = torch.cat([s, s.new_zeros(L, nq * 64 - N, G)], 1)
    s = s.reshape(L, nq, 4, 16, G)  # quad, r, row, block
    parts = []
    if nfull:
        sf = s[..., :4 * nfull].reshape(L, nq, 4, 16, nfull, 4)  # quad, r, row, c, kq
        parts.append(sf.permute(0, 1, 4, 5, 3, 2).reshape(L, nq, nfull * 256))
    if tq:
        st = s[..., 4 * nfull:]  # quad, r, row, kq
        parts.append(st.permute(0, 1, 4, 3, 2).reshape(L, nq, tq * 64))
    return torch.cat(parts, -1).contiguous()


def _unpack_scales(scale: torch.Tensor, N: int, G: int) -> torch.Tensor:
    """Inverse of _pack_scales: [L, ceil(N/64), 64G] -> [L, N, G]."""
    nq, nfull, tq = (N // 16 + 3) // 4, G // 4, G % 4
    s = scale.reshape(-1, nq, G * 64)
    L = s.shape[0]
    outs = []
    if nfull:
        sf = s[:, :, :nfull * 256].reshape(L, nq, nfull, 4, 16, 4)  # quad, c, kq, row, r
        outs.append(sf.permute(0, 1, 5, 4, 2, 3).reshape(L, nq, 4, 16, nfull * 4))
    if tq:
        st = s[:, :, nfull * 256:].reshape(L, nq, tq, 16, 4)  # quad, kq, row, r
        outs.append(st.permute(0, 1, 4, 3, 2))
    return torch.cat(outs, 4).reshape(L, nq * 64, G)[:, :N].contiguous()


def pack_mxfp8(codes: torch.Tensor, scales: torch.Tensor):
    """OCP MXFP8 codes [..., N, K/32, 32] (E4M3FN bytes) + scales [..., N, K/32] (E8M0) ->
    packed (data [..., N/16, 16K], scale [..., ceil(N/64), 2K]).

    data: chunk c of row group g at g*16K + c*2048, in two halves of 1 KiB (h = 0, 1:
    elements 16h .. 16h + 15 of each 32-block, the operands of MFMA steps 2h and 2h + 1);
    inside a half the 16 bytes of lane l are row 16g + l%16, K-block 4c + l//16.  A
    partial last chunk of tq < 4 blocks keeps halves of 256 tq bytes (lanes l < 16 tq).
    scale: as pack_mxfp4."""
    if codes.dtype != torch.uint8 or scales.dtype != torch.uint8:
        raise TypeError("MXFP8 codes and scales must be uint8")
    lead = codes.shape[:-3]
    N, G = codes.shape[-3], codes.shape[-2]
    if codes.shape[-1] != 32 or tuple(scales.shape) != tuple(codes.shape[:-1]):
        raise ValueError("expected codes [..., N, G, 32] and scales [..., N, G]")
    if N % 16:
        raise ValueError(f"row count {N} must be a multiple of 16")
    c = codes.reshape(-1, N // 16, 16, G, 2, 16)  # L, rg, r, block, half, byte
    L, nrg, nfull, tq = c.shape[0], N // 16, G // 4, G % 4
    parts = []
    if nfull:
        cf = c[:, :, :, :4 * nfull].reshape(L, nrg, 16, nfull, 4, 2, 16)  # r, chunk, q, h, byte
        parts.append(cf.permute(0, 1, 3, 5, 4, 2, 6).reshape(L, nrg, nfull * 2048))
    if tq:
        ct = c[:, :, :, 4 * nfull:]  # L, rg, r, tq, h, byte
        parts.append(ct.permute(0, 1, 4, 3, 2, 5).reshape(L, nrg, tq * 512))
    d = torch.cat(parts, -1).contiguous()
    sc = _pack_scales(scales.reshape(-1, N, G))
    return d.reshape(*lead, nrg, G * 512), sc.reshape(*lead, (N + 63) // 64, G * 64)


def unpack_mxfp8(data: torch.Tensor, scale: torch.Tensor):
    """Inverse of pack_mxfp8 -> codes [..., N, K/32, 32] and scales [..., N, K/32]."""
    lead = data.shape[:-2]
    nrg, nbytes = data.shape[-2], data.shape[-1]
    G = nbytes // 512
    nfull, tq = G // 4, G % 4
    d = data.reshape(-1, nrg, nbytes)
    L = d.shape[0]
    outs = []
    if nfull:
        df = d[:, :, :nfull * 2048].reshape(L, nrg, nfull, 2, 4, 16, 16)  # c, h, q, r, byte
        outs.append(df.permute(0, 1, 5, 2, 4, 3, 6).reshape(L, nrg, 16, nfull * 4, 2, 16))
    if tq:
        dt = d[:, :, nfull * 2048:].reshape(L, nrg, 2, tq, 16, 16)  # h, tq, r, byte
        outs.append(dt.permute(0, 1, 4, 3, 2, 5))
    c = torch.cat(outs, 3).reshape(*lead, nrg * 16, G, 32)
    sc = _unpack_scales(scale, nrg * 16, G).reshape(*lead, nrg * 16, G)
    return c.contiguous(), sc


def packed_scale_shape(N: int, K: int):
    """Trailing shape of the packed scale tensor of an [N, K] matrix."""
    return ((N + 63) // 64, 2 * K)


def unpack_mxfp4(data: torch.Tensor, scale: torch.Tensor):
    """Inverse of pack_mxfp4: packed [..., N/16, 8K] + [..., ceil(N/64), 2K] ->
    OCP blocks [..., N, K/32, 16] and scales [..., N, K/32]."""
    lead = data.shape[:-2]
    nrg, nbytes = data.shape[-2], data.shape[-1]
    G = nbytes // 256
    nfull, tq = G // 4, G % 4
    nq = (nrg + 3) // 4
    d = data.reshape(-1, nrg, nbytes)
    s = scale.reshape(-1, nq, G * 64)
    L = d.shape[0]
    outs_b, outs_s = [], []
    if nfull:
        bf = d[:, :, :nfull * 1024].reshape(L, nrg, nfull, 4, 16, 16)  # rg, c, q, r, byte
        outs_b.append(bf.permute(0, 1, 4, 2, 3, 5).reshape(L, nrg, 16, nfull * 4, 16))
        sf = s[:, :, :nfull * 256].reshape(L, nq, nfull, 4, 16, 4)  # quad, c, kq, row, r
        outs_s.append(sf.permute(0, 1, 5, 4, 2, 3).reshape(L, nq, 4, 16, nfull * 4))
    if tq:
        bt = d[:, :, nfull * 1024:].reshape(L, nrg, tq, 16, 16)  # rg, tq, r, byte
        outs_b.append(bt.permute(0, 1, 3, 2, 4))
        st = s[:, :, nfull * 256:].reshape(L, nq, tq, 16, 4)  # quad, kq, row, r
        outs_s.append(st.permute(0, 1, 4, 3, 2))
    b = torch.cat(outs_b, 3).reshape(*lead, nrg * 16, G, 16)
    sc = torch.cat(outs_s, 4).reshape(-1, nq * 64, G)[:, :nrg * 16]
    sc = sc.reshape(*lead, nrg * 16, G)
    return b.contiguous(), sc.contiguous()


def interleave_row_groups(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """[E, I, ...] gate and up rows -> [E, 2I, ...] alternating 16-row groups."""
    E, I = gate.shape[:2]
    rest = gate.shape[2:]
    g = gate.reshape(E, I // 16, 1, 16, *rest)
    u = up.reshape(E, I // 16, 1, 16, *rest)
    return torch.cat([g, u], 2).reshape(E, 2 * I, *rest)


def fuse_gate_up(gate_q: torch.Tensor, gate_s: torch.Tensor, up_q: torch.Tensor,
                 up_s: torch.Tensor):
    """Packed gate and up projections of one MLP (MXFP4 or MXFP8, each data [I/16, bytes]
    and scale [ceil(I/64), 2K]) -> the fused gate_up of an expert: data [2I/16, bytes] with
    gate and up 16-row groups alternating, scale [ceil(2I/64), 2K].  The data of a row group
    is self-contained, so the rows interleave as they are; scales are packed four row
    groups to a quad and are re-packed."""
    if gate_q.shape != up_q.shape or gate_s.shape != up_s.shape or gate_q.dim() != 2:
        raise ValueError(f"gate {tuple(gate_q.shape)}/{tuple(gate_s.shape)} and up "
                         f"{tuple(up_q.shape)}/{tuple(up_s.shape)} must be equal 2-D packed "
                         "tensors")
    nrg = gate_q.shape[0]
    G = gate_s.shape[1] // 64
    if gate_s.shape != ((nrg * 16 + 63) // 64, 64 * G):
        raise ValueError(f"scale shape {tuple(gate_s.shape)} does not match {nrg} row groups")
    data = torch.stack([gate_q, up_q], 1).reshape(2 * nrg, gate_q.shape[1]).contiguous()
    sg = _unpack_scales(gate_s, nrg * 16, G)
    su = _unpack_scales(up_s, nrg * 16, G)
    sc = interleave_row_groups(sg, su)  # [1, 2I, G]
    return data, _pack_scales(sc)[0]


def deinterleave_rows(t: torch.Tensor):
    """Checkpoint gate_up rows (2i = gate_i, 2i+1 = up_i) -> (gate, up) along dim 1."""
    return t[:, 0::2], t[:, 1::2]


def gate_up_bias_from_checkpoint(bias: torch.Tensor, up_offset: float = 1.0) -> torch.Tensor:
    """Checkpoint gate_up bias [E, 2I] (interleaved) -> [E, 2, I] = (gate, up + up_offset),
    the +1 added in the bias dtype as the reference loader does
    (weight_loaders_bf16.py:393-422; model_mxfp4.py:1104 passes hidden_act_bias=1.0)."""
    gate = bias[:, 0::2]
    up = bias[:, 1::2].clone()
    if up_offset:
        up = up + up_offset
    return torch.stack([gate, up], 1).contiguous()


@dataclass
class MXFP4Experts:
    """Packed expert weights of one MoE layer (all tensors on one device).

    gu_q [E, 2I/16, 8H], gu_s [E, ceil(2I/64), 2H]  fused gate_up (row groups alternate gate/up)
    dn_q [E, H/16, 8I],  dn_s [E, ceil(H/64), 2I]   down projection
    gu_bias [E, 2, I] bf16 (up half already holds +1 for GPT-OSS) or None
    dn_bias [E, H] bf16 or None
    """

    gu_q: torch.Tensor
    gu_s: torch.Tensor
    dn_q: torch.Tensor
    dn_s: torch.Tensor
    gu_bias: Optional[torch.Tensor]
    dn_bias: Optional[torch.Tensor]
    E: int
    H: int
    I: int

    @classmethod
    def from_split(cls, gate_blocks, gate_scales, up_blocks, up_scales, down_blocks, down_scales,
                   gu_bias=None, dn_bias=None):
        """gate/up blocks [E, I, H/32, 16] (+ scales [E, I, H/32]); down [E, H, I/32, 16]."""
        E, I, Gh = gate_blocks.shape[:3]
        H = Gh * 32
        gu_b = interleave_row_groups(gate_blocks, up_blocks)
        gu_sc = interleave_row_groups(gate_scales, up_scales)
        gu_q, gu_s = pack_mxfp4(gu_b, gu_sc)
        dn_q, dn_s = pack_mxfp4(down_blocks, down_scales)
        return cls(gu_q, gu_s, dn_q, dn_s, gu_bias, dn_bias, E, H, I)

    @classmethod
    def from_checkpoint(cls, gate_up_blocks, gate_up_scales, down_blocks, down_scales,
                        gate_up_bias=None, down_bias=None, up_bias_offset: float = 1.0):
        """HF GPT-OSS tensors (interleaved gate/up rows) -> packed experts."""
        gb, ub = deinterleave_rows(gate_up_blocks)
        gs, us = deinterleave_rows(gate_up_scales)
        gub = None if gate_up_bias is None else gate_up_bias_from_checkpoint(gate_up_bias,
                                                                             up_bias_offset)
        return cls.from_split(gb, gs, ub, us, down_blocks, down_scales, gub, down_bias)

    def to(self, device):
        mv = lambda t: None if t is None else t.to(device)  # noqa: E731
        return MXFP4Experts(mv(self.gu_q), mv(self.gu_s), mv(self.dn_q), mv(self.dn_s),
                            mv(self.gu_bias), mv(self.dn_bias), self.E, self.H, self.I)

    def nbytes_per_expert(self) -> int:
        n = (self.gu_q[0].numel() + self.gu_s[0].numel() + self.dn_q[0].numel()
             + self.dn_s[0].numel())
        if self.gu_bias is not None:
            n += self.gu_bias[0].numel() * self.gu_bias.element_size()
        if self.dn_bias is not None:
            n += self.dn_bias[0].numel() * self.dn_bias.element_size()
        return int(n)
