"""Fused decode MoE block (RMSNorm + router top-k + expert MLPs) on the MI355X kernels.

Mirrors vllm_neuron/functional/moe/moe_block_tkg.py:305-571 (signature, defaults,
exception types).  The reference runs nkilib moe_block_tkg (:469-517) or its torch
flow ``_torch_moe_block_tkg_impl`` (:56-302); here, with every expert on the rank,
one mxmoe_moe_block_decode call: RMSNorm (variance over the first ``hidden_actual``
columns, result cast to the input dtype as :134-150), the router on the normalized
rows (fp32 logits, router_pre_norm / norm_topk_prob as :152-204), then the experts (fp32
expert math over the selected experts, ascending-id fp32 sum, cast to the input dtype).
With a slice of the experts (rank_id), the same steps as mxmoe_rmsnorm,
mxmoe_router_topk and mxmoe_moe_tkg on the local expert ids.  bf16 expert weights (the
bf16 model's call, model_bf16.py:1199-1252: gate_up [E_L, H, 2, I], down [E_L, I, H])
take those steps with mxmoe_moe_tkg_bf16 for the experts.

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
from ._cache import transposed_rows
from ._common import act_code, require_mxfp4, resolve_experts, scale_code
from .moe_tkg import moe_tkg_bf16_raw, moe_tkg_raw
from .router import rms_norm, router_topk_raw


def rmsnorm(x: Tensor, gamma: Tensor, eps: float, hidden_actual: Optional[int] = None) -> Tensor:
    """The decode block's RMSNorm (moe_block_tkg.py:134-150): bf16 [T, H] -> bf16 [T, H],
    mean square over the first hidden_actual columns, the other columns zeroed."""
    return rms_norm(x, gamma, eps, hidden_actual, all_cols=False)


def _router_dtype_code(t: Tensor, what: str) -> int:
    return _lib.dtype_code(t.dtype, what, (torch.bfloat16, torch.float16))


def block_decode_raw(x, gamma, eps, hidden_actual, router_weights, bias, act, pre_norm, renorm,
                     top_k, ex, hidden_act, clamps, scale_mode, want_logits, want_idx=False):
    """mxmoe_moe_block_decode: x bf16 [T, H] (not normalized), router_weights [H, E]
    (bf16 or fp16), bias [E] or None, ex: packed experts holding every expert.
    Returns (out bf16 [T, H], logits fp32 [T, E] or None, topk_idx int32 [T, k] or None)."""
    dev = _lib.require_cuda(x, gamma, router_weights, ex.gu_q)
    E, H, I = ex.E, ex.H, ex.I
    T = x.shape[0]
    ha = H if hidden_actual is None else int(hidden_actual)
    g = gamma.reshape(-1).to(torch.float32).contiguous()
    if g.numel() != H:
        raise ValueError(f"gamma has {g.numel()} elements, expected {H}")
    if x.shape[1] != H:
        raise ValueError(f"hidden states have {x.shape[1]} columns, the experts {H}")
    w_eh = transposed_rows(router_weights)
    wdt = _router_dtype_code(w_eh, "router_weights")
    bdt = _lib.DT_BF16
    if bias is not None:
        bias = bias.reshape(-1).contiguous()
        bdt = _lib.dtype_code(bias.dtype, "router_bias")
    x = x.contiguous()
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    logits = torch.empty(T, E, dtype=torch.float32, device=dev) if want_logits else None
    idx = torch.empty(T, top_k, dtype=torch.int32, device=dev) if want_idx else None
    L = _lib.lib()
    ws = _lib.workspace(L.mxmoe_moe_block_decode_workspace_bytes(T, H, I, E, top_k), dev)
    rc = L.mxmoe_moe_block_decode(
        x.data_ptr(), g.data_ptr(), ha, float(eps), w_eh.data_ptr(), wdt, _lib.ptr(bias), bdt,
        act, int(pre_norm), int(renorm), 1e-20, ex.gu_q.data_ptr(), ex.gu_s.data_ptr(),
        ex.dn_q.data_ptr(), ex.dn_s.data_ptr(), _lib.ptr(ex.gu_bias), _lib.ptr(ex.dn_bias), T, H,
        I, E, top_k, hidden_act, clamps, scale_mode, out.data_ptr(), _lib.ptr(logits),
        _lib.ptr(idx), ws.data_ptr(), ws.numel(), None, _lib.stream_handle(dev))
    _lib.check(rc, "mxmoe_moe_block_decode")
    return out, logits, idx


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
    """inp bf16 [B, S, H] or [T, H]; gamma [1, H] or [H]; router_weights [H, E] (bf16 or
    fp16); router_bias [1, E] or [E]; expert weights packed (uint8), in the reference's
    Trainium MX layout (uint16 [E_L, 128, 2, H/512, I], converted once per tensor version)
    or bf16 ([E_L, H, 2, I] and [E_L, I, H]).
    Returns output [T, H] (+ router_logits [T, E] fp32).

    router_mm_dtype is accepted and leaves the arithmetic as the reference's torch flow
    has it: router logits in fp32 from the bf16 normalized rows and the router weights
    (moe_block_tkg.py:152-162, fp16 weights exactly as fp32)."""
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
    ex = resolve_experts(expert_gate_up_weights, expert_gate_up_weights_scale,
                         expert_down_weights, expert_down_weights_scale, expert_gate_up_bias,
                         expert_down_bias)
    bf16w = ex.fmt == _lib.WFMT_BF16
    if not bf16w:
        require_mxfp4(ex, "moe_block_tkg")
    E_L = ex.E
    fn = member_name(router_act_fn)
    if fn == "SOFTMAX":
        act = _lib.ROUTER_SOFTMAX
    elif fn == "SIGMOID":
        act = _lib.ROUTER_SIGMOID
    else:
        raise NotImplementedError(f"Router activation {fn} is not supported")
    _router_dtype_code(router_weights, "router_weights")
    E_g = router_weights.shape[1]
    bias = None if router_bias is None else router_bias.reshape(-1)
    if bias is not None and bias.numel() != E_g:
        raise ValueError(f"router_bias has {bias.numel()} elements, expected {E_g}")
    clamps = _lib.clamps_array(gate_clamp_lower_limit, gate_clamp_upper_limit,
                               up_clamp_lower_limit, up_clamp_upper_limit)
    if E_L == E_g and not bf16w:
        # Every expert on this rank: RMSNorm, router and experts in one library call.
        out, logits, _ = block_decode_raw(inp, gamma, eps, hidden_actual, router_weights, bias,
                                          act, bool(router_pre_norm), bool(norm_topk_prob),
                                          top_k, ex, act_code(hidden_act_fn), clamps,
                                          scale_code(expert_affinities_scaling_mode),
                                          not skip_router_logits)
        return out if skip_router_logits else (out, logits)
    xn = rmsnorm(inp, gamma, eps, hidden_actual)
    _, logits, idx, val = router_topk_raw(xn, transposed_rows(router_weights), top_k, bias, act,
                                          bool(router_pre_norm), bool(norm_topk_prob), 1e-20)
    if E_L < E_g and rank_id is not None:
        idx = idx - E_L * rank_id.reshape(-1)[0].to(idx.dtype)
    run = moe_tkg_bf16_raw if bf16w else moe_tkg_raw
    out = run(xn, idx, val, ex, act_code(hidden_act_fn), clamps,
              scale_code(expert_affinities_scaling_mode))
    if skip_router_logits:
        return out
    return out, logits
