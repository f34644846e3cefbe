"""Converter from vllm-neuron's Trainium MXFP4 kernel layout to this package's packed layout.

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
import os
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


# ---------------------------------------------------------------------------------------
# In-place conversion: no second copy of the experts in device memory.

_MARK = "_mxmoe_packed_in_place"
_in_place = os.environ.get("VLLM_NEURON_AMD_CONVERT_IN_PLACE", "0") == "1"


def set_convert_in_place(enabled: bool) -> bool:
    """Whether the MoE operators, handed Trainium-layout MXFP4 experts, rewrite them in
    place (``convert_in_place``) instead of keeping a converted copy.  Off by default (the
    caller's tensors then stay as they are); the environment variable
    ``VLLM_NEURON_AMD_CONVERT_IN_PLACE=1`` turns it on at import.  Returns the previous
    setting."""
    global _in_place
    prev, _in_place = _in_place, bool(enabled)
    return prev


def convert_in_place_enabled() -> bool:
    return _in_place


def _version(t: torch.Tensor):
    try:
        return t._version
    except RuntimeError:  # inference tensors keep no version counter
        return None


def owns_memory(t: torch.Tensor) -> bool:
    """Not a view, and alone in its storage: a version bump then means this tensor was
    written."""
    return (t._base is None and t.storage_offset() == 0 and t.is_contiguous()
            and t.untyped_storage().nbytes() == t.numel() * t.element_size())


def _packed_views(gu_w, gu_s, dn_w, dn_s, H_pad: int, I_pad: int):
    """The four tensors' bytes viewed as packed experts at the padded sizes."""
    E = gu_w.shape[0]

    def flat(t):
        return t.view(torch.uint8).reshape(-1)

    return (flat(gu_w).view(E, 2 * I_pad // 16, 8 * H_pad),
            flat(gu_s).view(E, (2 * I_pad + 63) // 64, 2 * H_pad),
            flat(dn_w).view(E, H_pad // 16, 8 * I_pad),
            flat(dn_s).view(E, (H_pad + 63) // 64, 2 * I_pad))


def packed_in_place(gate_up_blocks: torch.Tensor, gate_up_scales: torch.Tensor,
                    down_blocks: torch.Tensor, down_scales: torch.Tensor):
    """The packed views (gu_q, gu_s, dn_q, dn_s) of tensors that ``convert_in_place``
    rewrote, or None: None as well when any of them was written in place since (a reload
    in the Trainium layout bumps its version counter)."""
    ts = (gate_up_blocks, gate_up_scales, down_blocks, down_scales)
    marks = [getattr(t, _MARK, None) for t in ts]
    if any(m is None or m[0] != _version(t) or m[1] != marks[0][1] for t, m in zip(ts, marks)):
        return None
    return _packed_views(*ts, *marks[0][1])


def convert_in_place(gate_up_blocks: torch.Tensor, gate_up_scales: torch.Tensor,
                     down_blocks: torch.Tensor, down_scales: torch.Tensor):
    """Rewrite the reference's Trainium-layout MXFP4 expert tensors (the shapes of
    ``experts_from_neuron_layout``'s first four arguments) into this package's packed layout
    at the padded sizes H_pad, I_pad, expert by expert, and return the packed views
    (gu_q, gu_s, dn_q, dn_s) of the same memory.  Per expert both layouts take the same
    bytes (gate_up I_pad H_pad data and I_pad H_pad / 16 scale bytes, down half of each,
    the expert dim leading in both), so no second copy of the experts is kept: the
    temporaries are one expert's.  The tensors keep their shapes and dtypes; each is marked
    (an attribute with its version counter) so that the MoE operators take the packed views
    from then on (``packed_in_place``).  Anything else that reads these tensors afterwards
    sees packed bytes; a later in-place write to one of them (reloading it in the Trainium
    layout) clears the mark.  Each tensor must own its memory (not a view, alone in its
    storage: the reference's per-layer parameters are), so that its version counter tells
    whether it was written."""
    ts = (gate_up_blocks, gate_up_scales, down_blocks, down_scales)
    done = packed_in_place(*ts)
    if done is not None:
        return done
    if gate_up_blocks.dtype not in (torch.uint16, torch.int16) or gate_up_blocks.dim() != 5:
        raise TypeError("gate_up_blocks must be the 5-D uint16 Trainium-layout tensor")
    if gate_up_blocks.is_cuda and torch.cuda.is_current_stream_capturing():
        raise RuntimeError("convert_in_place under HIP graph capture: every replay would "
                           "rewrite the bytes again; convert before capturing")
    for t in ts:
        if not owns_memory(t):
            raise ValueError("in-place conversion needs tensors that own their memory "
                             "(contiguous, not views, alone in their storage)")
    E = gate_up_blocks.shape[0]
    H_pad = gate_up_blocks.shape[3] * 512
    I_pad = gate_up_scales.shape[4]
    views = _packed_views(*ts, H_pad, I_pad) if all(
        t.numel() * t.element_size() == n for t, n in zip(
            ts, (E * H_pad * I_pad, E * H_pad * I_pad // 16, E * H_pad * I_pad // 2,
                 E * H_pad * I_pad // 32))) else None
    if views is None:
        raise ValueError("tensor sizes do not match the Trainium layout at H_pad="
                         f"{H_pad}, I_pad={I_pad}")
    with torch.no_grad():
        for e in range(E):
            # expert e's packed bytes are materialized before they overwrite its Trainium ones
            ex = experts_from_neuron_layout(gate_up_blocks[e:e + 1], gate_up_scales[e:e + 1],
                                            down_blocks[e:e + 1], down_scales[e:e + 1], H_pad,
                                            I_pad)
            for v, p in zip(views, (ex.gu_q, ex.gu_s, ex.dn_q, ex.dn_s)):
                v[e].copy_(p[0])
    for t in ts:
        setattr(t, _MARK, (_version(t), (H_pad, I_pad)))
    return views
