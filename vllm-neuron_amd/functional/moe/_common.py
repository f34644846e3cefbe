"""Argument normalization shared by the expert-MLP entry points."""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from ... import _lib
from ...enums import member_name


def act_code(act) -> int:
    name = member_name(act)
    if name == "SiLU":
        return _lib.ACT_SILU
    if name == "GELU":
        return _lib.ACT_GELU
    if name == "Swish":
        return _lib.ACT_SWISH
    raise NotImplementedError(f"activation {name} has no MI355X kernel")


def scale_code(mode) -> int:
    name = member_name(mode)
    if name == "POST_SCALE":
        return _lib.SCALE_POST
    if name == "NO_SCALE":
        return _lib.SCALE_NO
    raise NotImplementedError(f"expert_affinities_scaling_mode {name} has no MI355X kernel")


def expert_shapes(gu_q: Tensor, gu_s: Tensor, dn_q: Tensor, dn_s: Tensor):
    """Packed weights -> (E, H, I), validating every shape."""
    for t, n in ((gu_q, "gate_up weight"), (gu_s, "gate_up scale"), (dn_q, "down weight"),
                 (dn_s, "down scale")):
        if t is None:
            raise AssertionError(f"{n} must be provided for MXFP4 compute")
        if t.dtype != torch.uint8 or t.dim() != 3:
            raise ValueError(f"{n}: expected a packed uint8 [E, rows/16, bytes] tensor, got "
                             f"{t.dtype} {tuple(t.shape)}")
    E = gu_q.shape[0]
    H = gu_q.shape[2] // 8
    I = gu_q.shape[1] * 16 // 2
    exp = {"gu_s": (E, (2 * I + 63) // 64, 2 * H), "dn_q": (E, H // 16, 8 * I),
           "dn_s": (E, (H + 63) // 64, 2 * I)}
    got = {"gu_s": tuple(gu_s.shape), "dn_q": tuple(dn_q.shape), "dn_s": tuple(dn_s.shape)}
    for k in exp:
        if exp[k] != got[k]:
            raise ValueError(f"packed weight shapes disagree: {k} is {got[k]}, expected {exp[k]}")
    return E, H, I


def gate_up_bias(b: Optional[Tensor], E: int, I: int) -> Optional[Tensor]:
    """[E, 2, I] or [E, 2I] ([gate | up]) bias -> contiguous bf16 [E, 2, I]."""
    if b is None:
        return None
    if b.numel() != E * 2 * I:
        raise ValueError(f"gate_up bias has {b.numel()} elements, expected {E * 2 * I}")
    if b.dtype != torch.bfloat16:
        raise NotImplementedError("gate_up bias must be bfloat16")
    return b.reshape(E, 2, I).contiguous()


def down_bias(b: Optional[Tensor], E: int, H: int) -> Optional[Tensor]:
    if b is None:
        return None
    if b.numel() != E * H:
        raise ValueError(f"down bias has {b.numel()} elements, expected {E * H}")
    if b.dtype != torch.bfloat16:
        raise NotImplementedError("down bias must be bfloat16")
    return b.reshape(E, H).contiguous()
