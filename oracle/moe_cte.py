"""Oracle: prefill expert MLP (``moe_cte`` torch fallback), dense and routed forms.

Test infrastructure only (see ``oracle/__init__.py``).

Follows vllm_neuron/functional/moe/moe_cte.py:
  * ``apply_activation`` <- ``_apply_activation`` (:423-445); Swish is
    ``g * sigmoid(1.702 g)`` with alpha fixed at :442
  * ``torch_moe_impl``   <- ``_torch_moe_impl`` (:448-581): all-expert bf16 einsums,
    bias, clamps, act(gate) * up, down einsum, bias, then the per-expert
    accumulation loop in ascending expert order (:572-579) where the fp32
    affinity promotes the running sum to fp32.

``torch_moe_impl_routed`` evaluates the same per-(token, expert) arithmetic only for
the experts a token selected.  Each token's row of a GEMM depends only on that
row, and unselected experts add ``y * 0.0 = 0`` to the running sum, so the two
agree whenever every expert output is finite; tests/test_oracle_moe.py checks the
routed form against the dense one on small shapes (the pin), and the dense form
against a float64 closed form of the SwiGLU/clamp algebra.
"""

from __future__ import annotations

from typing import Optional

import torch

SILU = "SiLU"
GELU = "GELU"
SWISH = "Swish"

POST_SCALE = "POST_SCALE"
PRE_SCALE = "PRE_SCALE"
PRE_SCALE_DELAYED = "PRE_SCALE_DELAYED"


def _name(v):
    return getattr(v, "name", v)


def apply_activation(g: torch.Tensor, act) -> torch.Tensor:
    """moe_cte.py:423-445."""
    act = _name(act)
    if act == SILU:
        return torch.nn.functional.silu(g)
    if act == GELU:
        return torch.nn.functional.gelu(g)
    if act == SWISH:
        return g * torch.sigmoid(g * 1.702)
    raise ValueError(f"Unsupported activation function: {act}")


def torch_moe_impl(hidden_states: torch.Tensor, expert_affinities: torch.Tensor,
                   gate_up_proj_weight: torch.Tensor, down_proj_weight: torch.Tensor,
                   gate_and_up_proj_bias: Optional[torch.Tensor] = None,
                   down_proj_bias: Optional[torch.Tensor] = None,
                   gate_clamp_upper_limit=None, gate_clamp_lower_limit=None,
                   up_clamp_upper_limit=None, up_clamp_lower_limit=None,
                   activation_function=SILU, expert_affinities_scaling_mode=POST_SCALE):
    """moe_cte.py:448-581.

    hidden [T(+1), H] bf16; affinities [T*E, 1]; gate_up [E, H, 2, I] bf16;
    down [E, I, H] bf16; gate_up bias [E, 2, I]; down bias [E, 1, H]."""
    mode = _name(expert_affinities_scaling_mode)
    E = gate_up_proj_weight.shape[0]
    H = hidden_states.shape[-1]
    dtype = hidden_states.dtype
    T = expert_affinities.shape[0] // E
    aff = expert_affinities.reshape(T, E)
    x = hidden_states[:T]
    gw = gate_up_proj_weight[:, :, 0, :]
    uw = gate_up_proj_weight[:, :, 1, :]
    if mode == PRE_SCALE:
        xs = x.unsqueeze(0) * aff.T.unsqueeze(-1)
        gate = torch.einsum("eth,ehi->eti", xs, gw)
        up = torch.einsum("eth,ehi->eti", xs, uw)
    else:
        gate = torch.einsum("th,ehi->eti", x, gw)
        up = torch.einsum("th,ehi->eti", x, uw)
    if gate_and_up_proj_bias is not None:
        gate = gate + gate_and_up_proj_bias[:, 0, :].unsqueeze(1)
        up = up + gate_and_up_proj_bias[:, 1, :].unsqueeze(1)
    if gate_clamp_lower_limit is not None or gate_clamp_upper_limit is not None:
        gate = gate.clamp(min=gate_clamp_lower_limit, max=gate_clamp_upper_limit)
    if up_clamp_lower_limit is not None or up_clamp_upper_limit is not None:
        up = up.clamp(min=up_clamp_lower_limit, max=up_clamp_upper_limit)
    inter = up * apply_activation(gate, activation_function)
    if mode == PRE_SCALE_DELAYED:
        inter = inter * aff.T.unsqueeze(-1)
    nxt = torch.einsum("eti,eih->eth", inter, down_proj_weight)
    if down_proj_bias is not None:
        nxt = nxt + down_proj_bias
    out = torch.zeros(T, H, dtype=dtype)
    if mode == POST_SCALE:
        for e in range(E):
            out = out + nxt[e] * aff[:, e:e + 1]
    else:
        for e in range(E):
            out = out + nxt[e]
    return out


def torch_moe_impl_routed(hidden_states, expert_affinities, gate_up_proj_weight,
                          down_proj_weight, gate_and_up_proj_bias=None, down_proj_bias=None,
                          gate_clamp_upper_limit=None, gate_clamp_lower_limit=None,
                          up_clamp_upper_limit=None, up_clamp_lower_limit=None,
                          activation_function=SILU, expert_affinities_scaling_mode=POST_SCALE,
                          token_rows=None):
    """Same arithmetic as ``torch_moe_impl`` for POST_SCALE, evaluated only on the
    (token, expert) pairs with non-zero affinity.  ``token_rows`` (optional 1-D
    index tensor) restricts the output to those tokens, which lets tests check a
    sample of a large batch.  Returns fp32 [len(rows), H]."""
    assert _name(expert_affinities_scaling_mode) == POST_SCALE
    E = gate_up_proj_weight.shape[0]
    H = hidden_states.shape[-1]
    T = expert_affinities.shape[0] // E
    aff = expert_affinities.reshape(T, E)
    rows = torch.arange(T) if token_rows is None else token_rows
    x = hidden_states[rows]
    a = aff[rows]
    out = torch.zeros(len(rows), H, dtype=hidden_states.dtype)
    # Per-expert terms, added in ascending expert order like :574-575.
    for e in range(E):
        sel = torch.nonzero(a[:, e] != 0).flatten()
        if sel.numel() == 0:
            continue
        xe = x[sel]
        g = xe @ gate_up_proj_weight[e, :, 0, :]
        u = xe @ gate_up_proj_weight[e, :, 1, :]
        if gate_and_up_proj_bias is not None:
            g = g + gate_and_up_proj_bias[e, 0, :]
            u = u + gate_and_up_proj_bias[e, 1, :]
        if gate_clamp_lower_limit is not None or gate_clamp_upper_limit is not None:
            g = g.clamp(min=gate_clamp_lower_limit, max=gate_clamp_upper_limit)
        if up_clamp_lower_limit is not None or up_clamp_upper_limit is not None:
            u = u.clamp(min=up_clamp_lower_limit, max=up_clamp_upper_limit)
        inter = u * apply_activation(g, activation_function)
        y = inter @ down_proj_weight[e]
        if down_proj_bias is not None:
            y = y + down_proj_bias[e].reshape(-1)
        term = torch.zeros(len(rows), H, dtype=torch.float32)
        term[sel] = y * a[sel, e:e + 1]
        out = out + term
    return out.to(torch.float32)
