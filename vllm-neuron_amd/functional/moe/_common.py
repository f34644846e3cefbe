"""Argument normalization shared by the expert-MLP entry points."""

from __future__ import annotations

from typing import NamedTuple, Optional

import torch
from torch import Tensor

from ... import _lib
from ...enums import member_name
from ...neuron_layout import (convert_in_place, convert_in_place_enabled,
                              experts_from_neuron_layout, owns_memory, packed_in_place,
                              unshuffle_hidden_dim, untile_gate_up_bias)
from ._cache import derived, discard


def act_code(act) -> int:
    name = member_name(act)
    if name == "SiLU":
        return _lib.ACT_SILU
    if name == "GELU":
        return _lib.ACT_GELU
    if name == "Swish":
        return _lib.ACT_SWISH
    raise NotImplementedError(f"activation {name} has no MI355X kernel")


def scale_code(mode, allow_no_scale: bool = True, allow_pre: bool = False) -> int:
    name = member_name(mode)
    if name == "POST_SCALE":
        return _lib.SCALE_POST
    if name == "NO_SCALE" and allow_no_scale:
        return _lib.SCALE_NO
    if name == "PRE_SCALE" and allow_pre:
        return _lib.SCALE_PRE
    if name == "PRE_SCALE_DELAYED" and allow_pre:
        return _lib.SCALE_PRE_DELAYED
    raise NotImplementedError(f"expert_affinities_scaling_mode {name} has no MI355X kernel")


def expert_shapes(gu_q: Tensor, gu_s: Tensor, dn_q: Tensor, dn_s: Tensor):
    """Packed weights -> (E, H, I, weight format), validating every shape.  The scales give
    H (2H bytes per quad row); the gate_up bytes per row group then tell MXFP4 (8H) from
    MXFP8 (16H)."""
    for t, n in ((gu_q, "gate_up weight"), (gu_s, "gate_up scale"), (dn_q, "down weight"),
                 (dn_s, "down scale")):
        if t is None:
            raise AssertionError(f"{n} must be provided for MXFP4 compute")
        if t.dtype != torch.uint8 or t.dim() != 3:
            raise ValueError(f"{n}: expected a packed uint8 [E, rows/16, bytes] tensor, got "
                             f"{t.dtype} {tuple(t.shape)}")
    E = gu_q.shape[0]
    H = gu_s.shape[2] // 2
    I = gu_q.shape[1] * 16 // 2
    if gu_q.shape[2] == 8 * H:
        fmt, per_k = _lib.WFMT_MXFP4, 8
    elif gu_q.shape[2] == 16 * H:
        fmt, per_k = _lib.WFMT_MXFP8, 16
    else:
        raise ValueError(f"gate_up weight: {gu_q.shape[2]} bytes per row group fit neither "
                         f"MXFP4 ({8 * H}) nor MXFP8 ({16 * H}) for H = {H}")
    exp = {"gu_s": (E, (2 * I + 63) // 64, 2 * H), "dn_q": (E, H // 16, per_k * I),
           "dn_s": (E, (H + 63) // 64, 2 * I)}
    got = {"gu_s": tuple(gu_s.shape), "dn_q": tuple(dn_q.shape), "dn_s": tuple(dn_s.shape)}
    for k in exp:
        if exp[k] != got[k]:
            raise ValueError(f"packed weight shapes disagree: {k} is {got[k]}, expected {exp[k]}")
    return E, H, I, fmt


def gate_up_bias(b: Optional[Tensor], E: int, I: int) -> Optional[Tensor]:
    """gate/up bias of packed experts: [E, 2, I] (gate, up) or [E, 2I] ([gate | up]) bf16
    -> contiguous [E, 2, I].  Any other shape raises: the reference's kernel-layout views
    ([E, I/4/n, 2, n, 4], model_mxfp4.py:1195-1201) belong to Trainium-layout weights."""
    if b is None:
        return None
    if tuple(b.shape) not in ((E, 2, I), (E, 2 * I)):
        raise ValueError(f"gate_up bias must be [{E}, 2, {I}] or [{E}, {2 * I}] for packed "
                         f"experts, got {tuple(b.shape)}")
    if b.dtype != torch.bfloat16:
        raise NotImplementedError("gate_up bias must be bfloat16")
    return b.reshape(E, 2, I).contiguous()


def down_bias(b: Optional[Tensor], E: int, H: int) -> Optional[Tensor]:
    """down bias of packed experts: [E, H] or [E, 1, H] bf16 -> contiguous [E, H]."""
    if b is None:
        return None
    if tuple(b.shape) not in ((E, H), (E, 1, H)):
        raise ValueError(f"down bias must be [{E}, {H}] or [{E}, 1, {H}] for packed experts, "
                         f"got {tuple(b.shape)}")
    if b.dtype != torch.bfloat16:
        raise NotImplementedError("down bias must be bfloat16")
    return b.reshape(E, H).contiguous()


class Experts(NamedTuple):
    gu_q: Tensor
    gu_s: Optional[Tensor]  # None for bf16 weights
    dn_q: Tensor
    dn_s: Optional[Tensor]
    gu_bias: Optional[Tensor]
    dn_bias: Optional[Tensor]
    E: int
    H: int
    I: int
    fmt: int = 0  # MXMOE_WFMT_*: 0 MXFP4, 1 MXFP8, 2 bf16


def is_bf16_weights(gate_up_weight: Tensor) -> bool:
    """Unquantized expert weights (the reference's shard_on_block operands)."""
    return gate_up_weight.is_floating_point()


def resolve_bf16_experts(gu_w: Tensor, dn_w: Tensor, gu_b: Optional[Tensor],
                         dn_b: Optional[Tensor]) -> Experts:
    """bf16 expert weights as moe_cte's shard_on_block takes them (moe_cte.py:117-124):
    gate_up [E, H, 2, I] (or the same memory as [E, H, 2I]: gate columns, then up), down
    [E, I, H]; biases [E, 2, I] (or [E, 2I]) and [E, H] (or [E, 1, H]).  Used in place
    (contiguous), no conversion."""
    for t, n in ((gu_w, "gate_up_proj_weight"), (dn_w, "down_proj_weight")):
        if t.dtype != torch.bfloat16:
            raise NotImplementedError(f"{n}: {t.dtype} expert weights have no MI355X kernel "
                                      "(bf16 or packed MX only)")
    if dn_w.dim() != 3:
        raise ValueError(f"down_proj_weight must be [E, I, H], got {tuple(dn_w.shape)}")
    E, I, H = dn_w.shape
    if tuple(gu_w.shape) not in ((E, H, 2, I), (E, H, 2 * I)):
        raise ValueError(f"gate_up_proj_weight must be [{E}, {H}, 2, {I}] (or [{E}, {H}, "
                         f"{2 * I}]) for down_proj_weight {tuple(dn_w.shape)}, got "
                         f"{tuple(gu_w.shape)}")
    gu, dn = gu_w.contiguous(), dn_w.contiguous()
    if gu.data_ptr() % 16 or dn.data_ptr() % 16:
        raise ValueError("bf16 expert weights must be 16-byte aligned")
    return Experts(gu, None, dn, None, gate_up_bias(gu_b, E, I), down_bias(dn_b, E, H), E, H, I,
                   _lib.WFMT_BF16)


def is_neuron_layout(gate_up_weight: Tensor) -> bool:
    """The reference's Trainium kernel layout: fp4 x4 packed in 16-bit words, 5-D."""
    return gate_up_weight.dtype in (torch.uint16, torch.int16) and gate_up_weight.dim() == 5


def _from_neuron_layout(gu_w, gu_s, dn_w, dn_s, gu_b, dn_b) -> Experts:
    """Weights in the layout of the reference's MXFP4 parameters (model_mxfp4.py:957-1018:
    gate_up [E, 128, 2, H/512, I] uint16 + scale [E, 16, 2, H/512, I] uint8, down
    [E, 128, I/512, H] uint16 + scale [E, 16, I/512, H] uint8, gate/up bias [E, 2I] in
    the tiled order (any view of it, e.g. the 5-D one of :1195-1201), down bias [E, H]
    with the hidden dim shuffled) -> packed experts at the padded sizes.  The padding
    the reference's loaders add is all zeros (codes, scales, biases), so the padded rows
    and columns add exact zeros.  Converted once per tensor version into a cached copy, or,
    with in-place conversion on (neuron_layout.set_convert_in_place) and tensors that own
    their memory, rewritten in place once and used as views from then on."""
    for t, n, d in ((gu_w, "gate_up weight", 5), (gu_s, "gate_up scale", 5),
                    (dn_w, "down weight", 4), (dn_s, "down scale", 4)):
        if t is None:
            raise AssertionError(f"{n} must be provided for MXFP4 compute")
        if t.dim() != d:
            raise ValueError(f"{n}: expected {d}-D kernel-layout tensor, got {tuple(t.shape)}")
    E = gu_w.shape[0]
    H_pad = gu_w.shape[3] * 512
    I_pad = gu_s.shape[4]
    exp = {"gate_up weight": (E, 128, 2, H_pad // 512, I_pad),
           "gate_up scale": (E, 16, 2, H_pad // 512, I_pad),
           "down scale": (E, dn_s.shape[1], dn_s.shape[2], H_pad)}
    got = {"gate_up weight": tuple(gu_w.shape), "gate_up scale": tuple(gu_s.shape),
           "down scale": tuple(dn_s.shape)}
    for k in exp:
        if exp[k] != got[k]:
            raise ValueError(f"kernel-layout shapes disagree: {k} is {got[k]}, expected {exp[k]}")
    if tuple(dn_w.shape) != (E, dn_s.shape[1] * 8, dn_s.shape[2], H_pad):
        raise ValueError(f"kernel-layout down weight {tuple(dn_w.shape)} does not match its "
                         f"scale {tuple(dn_s.shape)}")
    if gu_s.dtype != torch.uint8 or dn_s.dtype != torch.uint8:
        raise ValueError("MXFP4 scales must be uint8")
    if gu_b is not None and gu_b.numel() != E * 2 * I_pad:
        raise ValueError(f"gate_up bias has {gu_b.numel()} elements, expected {E * 2 * I_pad}")
    if dn_b is not None and dn_b.numel() != E * H_pad:
        raise ValueError(f"down bias has {dn_b.numel()} elements, expected {E * H_pad}")
    for b, n in ((gu_b, "gate_up bias"), (dn_b, "down bias")):
        if b is not None and b.dtype != torch.bfloat16:
            raise NotImplementedError(f"{n} must be bfloat16")

    packed = packed_in_place(gu_w, gu_s, dn_w, dn_s)
    # not while a HIP graph is being captured: its replays would rewrite the bytes again
    if packed is None and convert_in_place_enabled() and not (
            gu_w.is_cuda and torch.cuda.is_current_stream_capturing()) and all(
            owns_memory(t) for t in (gu_w, gu_s, dn_w, dn_s)):
        discard(gu_w)  # a converted copy made before is stale from here on
        packed = convert_in_place(gu_w, gu_s, dn_w, dn_s)
    if packed is not None:  # the caller's tensors hold the packed bytes: views, no copy
        gub = None if gu_b is None else derived(
            "neuron_gu_bias", (gu_b,),
            lambda: untile_gate_up_bias(gu_b.reshape(E, 2 * I_pad), I_pad).contiguous())
        dnb = None if dn_b is None else derived(
            "neuron_dn_bias", (dn_b,),
            lambda: unshuffle_hidden_dim(dn_b.reshape(E, H_pad), -1).contiguous())
        return Experts(*packed, gub, dnb, E, H_pad, I_pad)

    def make():
        ex = experts_from_neuron_layout(
            gu_w, gu_s, dn_w, dn_s, H_pad, I_pad,
            None if gu_b is None else gu_b.reshape(E, 2 * I_pad),
            None if dn_b is None else dn_b.reshape(E, H_pad))
        return Experts(ex.gu_q, ex.gu_s, ex.dn_q, ex.dn_s, ex.gu_bias, ex.dn_bias, E, H_pad,
                       I_pad)

    return derived("neuron_layout", (gu_w, gu_s, dn_w, dn_s, gu_b, dn_b), make)


def resolve_experts(gu_w: Tensor, gu_s: Optional[Tensor], dn_w: Tensor, dn_s: Optional[Tensor],
                    gu_b: Optional[Tensor], dn_b: Optional[Tensor]) -> Experts:
    """The expert arguments of moe_cte / moe_tkg / moe_block_tkg in any layout: this
    build's packed MXFP4 or MXFP8 (uint8, 3-D; biases [E, 2, I] and [E, H]), the reference's
    Trainium kernel layout (converted once per tensor version, see _from_neuron_layout), or
    bf16 weights (see resolve_bf16_experts; scales must then be absent)."""
    if is_bf16_weights(gu_w):
        if gu_s is not None or dn_s is not None:
            raise NotImplementedError("scaled (FP8) shard_on_block weights have no MI355X "
                                      "kernel: bf16 weights take no scales")
        return resolve_bf16_experts(gu_w, dn_w, gu_b, dn_b)
    if is_neuron_layout(gu_w):
        return _from_neuron_layout(gu_w, gu_s, dn_w, dn_s, gu_b, dn_b)
    E, H, I, fmt = expert_shapes(gu_w, gu_s, dn_w, dn_s)
    return Experts(gu_w, gu_s, dn_w, dn_s, gate_up_bias(gu_b, E, I), down_bias(dn_b, E, H), E,
                   H, I, fmt)


def require_mxfp4(ex: Experts, what: str) -> None:
    """The decode operators take MXFP4 experts only, as the reference's decode kernel does
    (vllm_neuron/functional/moe/moe_tkg.py:48: "Currently only supports MXFP4 on Trn3")."""
    if ex.fmt != _lib.WFMT_MXFP4:
        kind = "bf16" if ex.fmt == _lib.WFMT_BF16 else "MXFP8"
        raise NotImplementedError(f"{what}: {kind} expert weights are supported by moe_cte only "
                                  "(the reference decode kernel supports MXFP4 only)")
