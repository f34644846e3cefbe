"""Oracle: dense MLP (``mlp`` torch fallback).

Test infrastructure only (see ``oracle/__init__.py``).

Follows vllm_neuron/functional/mlp.py:
  * ``activation_fn`` <- ``_get_activation_fn`` (:261-286): SiLU and Swish both map to
    ``torch.nn.functional.silu`` (:278-279; unlike moe_cte, whose Swish is GPT-OSS's
    ``g * sigmoid(1.702 g)``), GELU to the exact erf form, GELU_Tanh_Approx to tanh
  * ``torch_mlp_impl`` <- ``_torch_mlp_impl`` (:313-418) without normalization or fused
    residual add (NormType.NO_NORM): ``gate = x @ gate_w (+ gate_b)``, ``up = x @ up_w
    (+ up_b)``, ``act(gate) * up``, ``@ down_w (+ down_b)``, every step on the tensors'
    own dtype (bf16 results, rounded once per op).

The reference flow has no clamps (the clamp limits reach only its device kernel); the
clamped variant here (``clamps``) applies them after the biases as ``_torch_moe_impl``
does (moe_cte.py:545-549), which is what the MI355X path computes; its placement is
pinned by the moe_cte flow, not by a dense-MLP one.

Pinned by tests/test_oracle_mlp.py: against ``oracle.moe_cte.torch_moe_impl`` with one
expert and affinity 1 (a separate restatement of a different reference function, with
the same per-op roundings), and against a float64 closed form for zero gate weights
(gate = gate_b, so out = (act(gate_b) * (x @ up_w + up_b)) @ down_w + down_b); the
Swish -> silu mapping against ``torch.nn.functional.silu``.
"""

from __future__ import annotations

from typing import Optional

import torch

SILU = "SiLU"
GELU = "GELU"
GELU_TANH = "GELU_Tanh_Approx"
SWISH = "Swish"


def _name(v):
    return getattr(v, "name", v)


def activation_fn(act):
    """mlp.py:261-286."""
    act = _name(act)
    if act in (SILU, SWISH):
        return torch.nn.functional.silu
    if act == GELU:
        return torch.nn.functional.gelu
    if act == GELU_TANH:
        return lambda x: torch.nn.functional.gelu(x, approximate="tanh")
    raise ValueError(f"Unsupported activation function: {act}")


def torch_mlp_impl(hidden: torch.Tensor, gate_w: torch.Tensor, up_w: torch.Tensor,
                   down_w: torch.Tensor, act=SILU, gate_b: Optional[torch.Tensor] = None,
                   up_b: Optional[torch.Tensor] = None, down_b: Optional[torch.Tensor] = None,
                   clamps=None) -> torch.Tensor:
    """mlp.py:371-418 (NO_NORM, no fused add, skip_gate False).

    hidden [T, H]; gate_w, up_w [H, I]; down_w [I, H]; biases [1, I] / [1, H] (all one
    dtype, bf16 in the tests).  ``clamps`` = (gate_lo, gate_hi, up_lo, up_hi) or None."""
    x = hidden
    gate = x @ gate_w
    if gate_b is not None:
        gate = gate + gate_b
    up = x @ up_w
    if up_b is not None:
        up = up + up_b
    if clamps is not None:
        g_lo, g_hi, u_lo, u_hi = clamps
        if g_lo is not None or g_hi is not None:
            gate = gate.clamp(min=g_lo, max=g_hi)
        if u_lo is not None or u_hi is not None:
            up = up.clamp(min=u_lo, max=u_hi)
    activated = activation_fn(act)(gate) * up
    out = activated @ down_w
    if down_b is not None:
        out = out + down_b
    return out
