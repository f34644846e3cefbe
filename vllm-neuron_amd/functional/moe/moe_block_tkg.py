"""Fused decode MoE block (RMSNorm + router top-k + expert MLPs) on the MI355X kernels.

Mirrors vllm_neuron/functional/moe/moe_block_tkg.py:305-571 (signature, defaults,
exception types).  The reference runs nkilib moe_block_tkg (:469-517) or its torch
flow ``_torch_moe_block_tkg_impl`` (:56-302); here: mxmoe_rmsnorm (variance over
the first ``hidden_actual`` columns, result cast to the input dtype as :134-150),
mxmoe_router_topk on the normalized rows (fp32 logits, router_pre_norm /
norm_topk_prob as :152-204), then mxmoe_moe_tkg (fp32 expert math over the
selected experts, ascending-id fp32 sum, cast to the input dtype).

Shared experts, fused residual add and activation quantization have no MI355X
kernel and raise NotImplementedError, like the reference's torch flow does for
most of them (:519-545).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from ... import _lib
from ...enums import ActFnType, ExpertAffinityScaleMode, RouterActFnType, member_name
from ._common import act_code, down_bias, expert_shapes, gate_up_bias, scale_code
from .moe_tkg import moe_tkg_raw
from .router import router_topk_raw


def rmsnorm(x: Tensor, gamma: Tensor, eps: float, hidden_actual: Optional[int] = None) -> Tensor:
    """bf16 [T, H] -> bf16 [T, H] with columns >= hidden_actual zeroed."""
    dev = _lib.require_cuda(x, gamma)
    T, H = x.shape
    ha = H if hidden_actual is None else int(hidden_actual)
    g = gamma.reshape(-1).to(torch.float32).contiguous()
    if g.numel() != H:
        raise ValueError(f"gamma has {g.numel()} elements, expected {H}")
    out = torch.empty_like(x)
    rc = _lib.lib().mxmoe_rmsnorm(x.contiguous().data_ptr(), g.data_ptr(), T, H, ha, float(eps),
                                  out.data_ptr(), _lib.stream_handle(dev))
    _lib.check(rc, "mxmoe_rmsnorm")
    return out


def moe_block_tkg(inp: Tensor, gamma: Tensor, router_weights: Tensor,
                  expert_gate_up_weights: Tensor, expert_down_weights: Tensor,
                  rank_id: Optional[Tensor] = None, top_k: int = 1,
                  shared_expert_gate_w: Optional[Tensor] = None,
                  shared_expert_up_w: Optional[Tensor] = None,
                  shared_expert_down_w: Optional[Tensor] = None,
                  expert_gate_up_weights_scale: Optional[Tensor] = None,
                  expert_down_weights_scale: Optional[Tensor] = None,
                  router_bias: Optional[Tensor] = None,
                  expert_gate_up_bias: Optional[Tensor] = None,
                  expert_down_bias: Optional[Tensor] = None,
                  shared_expert_gate_bias: Optional[Tensor] = None,
                  shared_expert_up_bias: Optional[Tensor] = None,
                  shared_expert_down_bias: Optional[Tensor] = None, eps: float = 1e-6,
                  router_act_fn=RouterActFnType.SIGMOID, router_pre_norm: bool = True,
                  norm_topk_prob: bool = False,
                  expert_affinities_scaling_mode=ExpertAffinityScaleMode.NO_SCALE,
                  hidden_act_fn=ActFnType.SiLU, hidden_act_scale_factor: Optional[float] = None,
                  hidden_act_bias: Optional[float] = None,
                  gate_clamp_upper_limit: Optional[float] = None,
                  gate_clamp_lower_limit: Optional[float] = None,
                  up_clamp_upper_limit: Optional[float] = None,
                  up_clamp_lower_limit: Optional[float] = None, router_mm_dtype=None,
                  hidden_actual: Optional[int] = None, skip_router_logits: bool = False,
                  is_all_expert: bool = False,
                  residual: Optional[Tensor] = None) -> Tuple[Tensor, ...]:
    """inp bf16 [B, S, H] or [T, H]; gamma [1, H] or [H]; router_weights bf16 [H, E];
    packed expert weights [E_L, ...].  Returns output [T, H] (+ router_logits [T, E])."""
    if shared_expert_gate_w is not None or shared_expert_down_w is not None or \
            shared_expert_up_w is not None:
        raise NotImplementedError("Shared experts have no MI355X kernel")
    if residual is not None:
        raise NotImplementedError("Fused residual add has no MI355X kernel")
    if hidden_act_scale_factor is not None or hidden_act_bias is not None:
        raise NotImplementedError(
            "hidden_act_scale_factor and hidden_act_bias are placeholders and must be None.")
    if inp.dim() == 3:
        inp = inp.reshape(-1, inp.shape[-1])
    if inp.dtype != torch.bfloat16:
        raise NotImplementedError("inp must be bfloat16")
    E_L, H, I = expert_shapes(expert_gate_up_weights, expert_gate_up_weights_scale,
                              expert_down_weights, expert_down_weights_scale)
    fn = member_name(router_act_fn)
    if fn == "SOFTMAX":
        act = _lib.ROUTER_SOFTMAX
    elif fn == "SIGMOID":
        act = _lib.ROUTER_SIGMOID
    else:
        raise NotImplementedError(f"Router activation {fn} is not supported")
    if router_weights.dtype != torch.bfloat16:
        raise NotImplementedError("router_weights must be bfloat16")
    if router_bias is not None and router_bias.dtype != torch.bfloat16:
        raise NotImplementedError("router_bias must be bfloat16")
    xn = rmsnorm(inp, gamma, eps, hidden_actual)
    w_eh = router_weights.t()
    bias = None if router_bias is None else router_bias.reshape(-1)
    _, logits, idx, val = router_topk_raw(xn, w_eh, top_k, bias, act, bool(router_pre_norm),
                                          bool(norm_topk_prob), 1e-20)
    E_g = router_weights.shape[1]
    if E_L < E_g and rank_id is not None:
        idx = idx - E_L * rank_id.reshape(-1)[0].to(idx.dtype)
    out = moe_tkg_raw(xn, idx, val, expert_gate_up_weights, expert_gate_up_weights_scale,
                      expert_down_weights, expert_down_weights_scale,
                      gate_up_bias(expert_gate_up_bias, E_L, I),
                      down_bias(expert_down_bias, E_L, H), act_code(hidden_act_fn),
                      _lib.clamps_array(gate_clamp_lower_limit, gate_clamp_upper_limit,
                                        up_clamp_lower_limit, up_clamp_upper_limit),
                      scale_code(expert_affinities_scaling_mode))
    if skip_router_logits:
        return out
    return out, logits
