"""Fused decode MoE block (RMSNorm + router top-k + expert MLPs) on the MI355X kernels.

Mirrors vllm_neuron/functional/moe/moe_block_tkg.py:305-571 (signature, defaults,
exception types).  The reference runs nkilib moe_block_tkg (:469-517) or its torch
flow ``_torch_moe_block_tkg_impl`` (:56-302); here, with every expert on the rank,
one mxmoe_moe_block_decode call: RMSNorm (variance over the first ``hidden_actual``
columns, result cast to the input dtype as :134-150), the router on the normalized
rows (fp32 logits, router_pre_norm / norm_topk_prob as :152-204), then the experts (fp32
expert math over the selected experts, ascending-id fp32 sum, cast to the input dtype).
With a slice of the experts (rank_id), the same steps as mxmoe_rmsnorm,
mxmoe_router_topk and mxmoe_moe_tkg on the local expert ids.

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


# The router weights arrive as [H, E] (the reference's layout); the kernels read [E, H].
# The transposed copy is kept per (storage, version, shape, strides), so a weight tensor
# passed at every decode step is transposed once (an in-place update bumps its version).
_ROUTER_T: "dict" = {}
_ROUTER_T_MAX = 256


def _router_eh(router_weights: Tensor) -> Tensor:
    key = (router_weights.data_ptr(), router_weights._version, tuple(router_weights.shape),
           tuple(router_weights.stride()), str(router_weights.device))
    w = _ROUTER_T.get(key)
    if w is None:
        if len(_ROUTER_T) >= _ROUTER_T_MAX:
            _ROUTER_T.clear()
        w = router_weights.t().contiguous()
        _ROUTER_T[key] = w
    return w


def _block_decode(x, gamma, eps, hidden_actual, router_weights, bias, act, pre_norm, renorm,
                  top_k, gu_q, gu_s, dn_q, dn_s, gub, dnb, hidden_act, clamps, scale_mode,
                  want_logits):
    """mxmoe_moe_block_decode: x bf16 [T, H] (not normalized), router_weights [H, E]."""
    dev = _lib.require_cuda(x, gamma, router_weights, gu_q)
    E, H, I = expert_shapes(gu_q, gu_s, dn_q, dn_s)
    T = x.shape[0]
    ha = H if hidden_actual is None else int(hidden_actual)
    g = gamma.reshape(-1).to(torch.float32).contiguous()
    if g.numel() != H:
        raise ValueError(f"gamma has {g.numel()} elements, expected {H}")
    if x.shape[1] != H:
        raise ValueError(f"hidden states have {x.shape[1]} columns, the experts {H}")
    w_eh = _router_eh(router_weights)
    if bias is not None:
        bias = bias.contiguous()
    x = x.contiguous()
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    logits = torch.empty(T, E, dtype=torch.float32, device=dev) if want_logits else None
    L = _lib.lib()
    ws = _lib.workspace(L.mxmoe_moe_block_decode_workspace_bytes(T, H, I, E, top_k), dev)
    rc = L.mxmoe_moe_block_decode(
        x.data_ptr(), g.data_ptr(), ha, float(eps), w_eh.data_ptr(), _lib.ptr(bias), act,
        int(pre_norm), int(renorm), 1e-20, gu_q.data_ptr(), gu_s.data_ptr(), dn_q.data_ptr(),
        dn_s.data_ptr(), _lib.ptr(gub), _lib.ptr(dnb), T, H, I, E, top_k, hidden_act, clamps,
        scale_mode, out.data_ptr(), _lib.ptr(logits), ws.data_ptr(), ws.numel(), None,
        _lib.stream_handle(dev))
    _lib.check(rc, "mxmoe_moe_block_decode")
    return out, logits


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
    E_g = router_weights.shape[1]
    bias = None if router_bias is None else router_bias.reshape(-1)
    if E_L == E_g:
        # Every expert on this rank: RMSNorm, router and experts in one library call.
        out, logits = _block_decode(inp, gamma, eps, hidden_actual, router_weights, bias, act,
                                    bool(router_pre_norm), bool(norm_topk_prob), top_k,
                                    expert_gate_up_weights, expert_gate_up_weights_scale,
                                    expert_down_weights, expert_down_weights_scale,
                                    gate_up_bias(expert_gate_up_bias, E_L, I),
                                    down_bias(expert_down_bias, E_L, H), act_code(hidden_act_fn),
                                    _lib.clamps_array(gate_clamp_lower_limit,
                                                      gate_clamp_upper_limit,
                                                      up_clamp_lower_limit,
                                                      up_clamp_upper_limit),
                                    scale_code(expert_affinities_scaling_mode),
                                    not skip_router_logits)
        return out if skip_router_logits else (out, logits)
    xn = rmsnorm(inp, gamma, eps, hidden_actual)
    w_eh = router_weights.t()
    _, logits, idx, val = router_topk_raw(xn, w_eh, top_k, bias, act, bool(router_pre_norm),
                                          bool(norm_topk_prob), 1e-20)
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
