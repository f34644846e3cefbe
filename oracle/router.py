"""Oracle: MoE router (linear -> top-k -> activation -> scatter), torch flow.

Test infrastructure only (see ``oracle/__init__.py``).

Follows vllm_neuron/functional/moe/router.py:
  * ``router``                       <- torch branch of ``router`` (:71-297) with
                                        ``_validate_router_inputs`` (:601-677)
  * ``topk_act_scatter``             <- ``_torch_router_impl_prenorm_linear_topk_act_scatter`` (:383-440)
  * ``act_topk_renorm_scatter``      <- ``_torch_router_impl_prenorm_linear_act_topk_renorm_scatter`` (:443-503)
  * ``topk_scatter_act``             <- ``_torch_router_impl_prenorm_linear_topk_scatter_act`` (:506-565)
  * ``apply_activation``             <- ``_apply_activation`` (:568-598)
  * ``rms_norm``                     <- ``_torch_rms_norm`` (:680-687)

Pinned by (tests/test_oracle_router.py): an fp64 brute force (per-token sorted
logits, Python ``math.exp`` softmax over the selected k) on small inputs, the
invariants (exactly k non-zeros per row, rows sum to 1 for softmax, selected
logits dominate unselected ones) and the lower-index-first order on hand-built ties.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

PRENORM_LINEAR_TOPK_ACT_SCATTER = "prenorm_linear_topk_act_scatter"
PRENORM_LINEAR_ACT_TOPK_RENORM_SCATTER = "prenorm_linear_act_topk_renorm_scatter"
PRENORM_LINEAR_TOPK_SCATTER_ACT = "prenorm_linear_topk_scatter_act"


def apply_activation(activation, x: torch.Tensor) -> torch.Tensor:
    """router.py:568-598.  A 16-bit x is activated in fp32 and rounded once to its
    dtype, the arithmetic of torch's CPU softmax / sigmoid on half tensors."""
    if activation == "softmax":
        return F.softmax(x.float(), dim=-1).to(x.dtype)
    if activation == "sigmoid":
        return torch.sigmoid(x.float()).to(x.dtype)
    if callable(activation):
        return activation(x)
    raise ValueError(f"Unsupported activation function: {activation}")


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """router.py:680-687."""
    dt = x.dtype
    x32 = x.to(torch.float32)
    var = x32.pow(2).mean(dim=-1, keepdim=True)
    return (x32 * torch.rsqrt(var + eps) * weight).to(dt)


def _logits(x, w_he, bias, gamma, eps, cdt):
    """router.py:422-426: F.linear of the operands cast to cdt.  For a 16-bit cdt it is
    written out as what torch's CPU linear computes on the reference platform: the cast
    operands' products summed in fp32, the cast bias added in fp32, one rounding to cdt
    (bit-identical to F.linear on 99.8 % of outputs there, one rounding step apart on
    the rest; the rounding of a half-precision CPU GEMM otherwise depends on the host's
    BLAS path)."""
    if gamma is not None:
        x = rms_norm(x, gamma, eps)
    if cdt == torch.float32:
        return F.linear(x.to(cdt), w_he.T.to(cdt), bias.to(cdt) if bias is not None else None)
    acc = x.to(cdt).float() @ w_he.to(cdt).float()
    if bias is not None:
        acc = acc + bias.to(cdt).float()
    return acc.to(cdt)


def topk_act_scatter(x, w_he, k, bias=None, activation="softmax", gamma=None, eps=1e-6,
                     computation_dtype=torch.float32):
    """router.py:383-440: logits -> topk (sorted, descending) -> act over the k
    selected values -> scatter into zeros [T, E]."""
    T = x.shape[0]
    E = w_he.shape[1]
    logits = _logits(x, w_he, bias, gamma, eps, computation_dtype)
    vals, idx = torch.topk(logits, k, dim=-1)
    probs = apply_activation(activation, vals)
    aff = torch.zeros(T, E, dtype=computation_dtype)
    aff.scatter_(1, idx, probs)
    return aff, logits


def act_topk_renorm_scatter(x, w_he, k, bias=None, activation="softmax", gamma=None,
                            eps=1e-6, computation_dtype=torch.float32):
    """router.py:443-503: act over all logits -> topk -> L1 renorm -> scatter."""
    T = x.shape[0]
    E = w_he.shape[1]
    logits = _logits(x, w_he, bias, gamma, eps, computation_dtype)
    probs = apply_activation(activation, logits)
    vals, idx = torch.topk(probs, k, dim=-1)
    # sum and quotient in fp32, each rounded once to cdt (torch's half-tensor CPU ops)
    s = vals.float().sum(dim=-1, keepdim=True).to(vals.dtype)
    vals = (vals.float() / s.float()).to(vals.dtype)
    aff = torch.zeros(T, E, dtype=computation_dtype)
    aff.scatter_(1, idx, vals)
    return aff, logits


def topk_scatter_act(x, w_he, k, bias=None, activation="softmax", gamma=None, eps=1e-6,
                     computation_dtype=torch.float32):
    """router.py:506-565: topk on raw logits -> scatter into -inf -> act over the row."""
    T = x.shape[0]
    E = w_he.shape[1]
    logits = _logits(x, w_he, bias, gamma, eps, computation_dtype)
    vals, idx = torch.topk(logits, k, dim=-1)
    aff = torch.full((T, E), float("-inf"), dtype=computation_dtype)
    aff.scatter_(1, idx, vals)
    return apply_activation(activation, aff), logits


_ORDERS = {
    PRENORM_LINEAR_TOPK_ACT_SCATTER: topk_act_scatter,
    PRENORM_LINEAR_ACT_TOPK_RENORM_SCATTER: act_topk_renorm_scatter,
    PRENORM_LINEAR_TOPK_SCATTER_ACT: topk_scatter_act,
}


def router(hidden_states: torch.Tensor, router_weights: torch.Tensor, top_k: int,
           router_bias: Optional[torch.Tensor] = None, activation="softmax",
           return_logits: bool = False, gamma: Optional[torch.Tensor] = None,
           eps: float = 1e-6, computation_dtype=torch.float32,
           router_computation_order: str = PRENORM_LINEAR_TOPK_ACT_SCATTER):
    """router.py:71-297 (torch branch): validate, cast x to computation_dtype, dispatch."""
    if hidden_states.dim() != 2 or router_weights.dim() != 2:
        raise ValueError("hidden_states and router_weights must be 2D")
    T, H = hidden_states.shape
    H_w, E = router_weights.shape
    if H != H_w:
        raise ValueError(f"Hidden dimension mismatch: {H} vs {H_w}")
    if top_k < 1 or top_k > E:
        raise ValueError(f"top_k must be between 1 and {E}, got {top_k}")
    x = hidden_states.to(computation_dtype)
    order = getattr(router_computation_order, "value", router_computation_order)
    aff, logits = _ORDERS[order](
        x, router_weights, top_k, router_bias, activation, gamma, eps, computation_dtype)
    return (aff, logits) if return_logits else aff
