"""Decode expert MLP given routing (token generation) on the MI355X kernel.

Mirrors vllm_neuron/functional/moe/moe_tkg.py:16-194.  The reference has no CPU
flow for this op (:191-194 raises for non-MXFP4 weights); its arithmetic is the
expert part of the moe_block_tkg torch flow (moe_block_tkg.py:223-297): fp32
gate/up, clamps, activation, fp32 down, weighted sum over the selected experts in
ascending id.  Here mxmoe_moe_tkg streams only the experts the batch selected.

is_all_expert and mask_unselected_experts do not change results (unselected
experts carry zero affinity) and select no separate code path.  Expert ids are
global; with ``rank_id`` the local range [E_L * rank, E_L * (rank + 1)) is kept
(expert parallelism), other ids are skipped.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from ... import _lib
from ...enums import ExpertAffinityScaleMode, MoEAllToAllVStrategy, member_name
from ._common import Experts, act_code, require_mxfp4, resolve_experts, scale_code


def moe_tkg_raw(x: Tensor, topk_idx: Tensor, topk_val: Tensor, ex: Experts, act: int, clamps,
                scale_mode: int, stage_events=None) -> Tensor:
    """Kernel call: x bf16 [T, H], topk_idx int32 [T, k] (local ids), topk_val fp32 [T, k],
    ex packed experts.  stage_events: optional 5 torch.cuda.Event recorded around routing,
    gate_up, down and combine."""
    dev = _lib.require_cuda(x, topk_idx, topk_val, ex.gu_q)
    E, H, I = ex.E, ex.H, ex.I
    if x.dim() != 2 or x.shape[1] != H:
        raise ValueError(f"hidden states must be [T, {H}], got {tuple(x.shape)}")
    T, K = topk_idx.shape
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    L = _lib.lib()
    ws = _lib.workspace(L.mxmoe_moe_tkg_workspace_bytes(T, H, I, E, K), dev)
    rc = L.mxmoe_moe_tkg(x.contiguous().data_ptr(), topk_idx.contiguous().data_ptr(),
                         topk_val.contiguous().data_ptr(), ex.gu_q.data_ptr(), ex.gu_s.data_ptr(),
                         ex.dn_q.data_ptr(), ex.dn_s.data_ptr(), _lib.ptr(ex.gu_bias),
                         _lib.ptr(ex.dn_bias), T, H, I, E, K, act, clamps, scale_mode,
                         out.data_ptr(), ws.data_ptr(), ws.numel(),
                         _lib.event_array(stage_events), _lib.stream_handle(dev))
    _lib.check(rc, "mxmoe_moe_tkg")
    return out


def moe_tkg_bf16_raw(x: Tensor, topk_idx: Tensor, topk_val: Tensor, ex: Experts, act: int,
                     clamps, scale_mode: int) -> Tensor:
    """mxmoe_moe_tkg_bf16: the same decode flow on bf16 experts (gate_up [E, H, 2, I], down
    [E, I, H]), as moe_block_tkg runs it for the bf16 model (model_bf16.py:1199-1252)."""
    dev = _lib.require_cuda(x, topk_idx, topk_val, ex.gu_q)
    E, H, I = ex.E, ex.H, ex.I
    if x.dim() != 2 or x.shape[1] != H:
        raise ValueError(f"hidden states must be [T, {H}], got {tuple(x.shape)}")
    T, K = topk_idx.shape
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    L = _lib.lib()
    ws = _lib.workspace(L.mxmoe_moe_tkg_bf16_workspace_bytes(T, H, I, E, K), dev)
    rc = L.mxmoe_moe_tkg_bf16(x.contiguous().data_ptr(), topk_idx.contiguous().data_ptr(),
                              topk_val.contiguous().data_ptr(), ex.gu_q.data_ptr(),
                              ex.dn_q.data_ptr(), _lib.ptr(ex.gu_bias), _lib.ptr(ex.dn_bias), T,
                              H, I, E, K, act, clamps, scale_mode, out.data_ptr(), ws.data_ptr(),
                              ws.numel(), _lib.stream_handle(dev))
    _lib.check(rc, "mxmoe_moe_tkg_bf16")
    return out


def moe_tkg(hidden_input: Tensor, expert_gate_up_weights: Tensor, expert_down_weights: Tensor,
            expert_affinities: Tensor, expert_index: Tensor, is_all_expert: bool,
            rank_id: Optional[Tensor] = None, expert_gate_up_bias: Optional[Tensor] = None,
            expert_down_bias: Optional[Tensor] = None,
            expert_gate_up_weights_scale: Optional[Tensor] = None,
            expert_down_weights_scale: Optional[Tensor] = None,
            hidden_input_scale: Optional[Tensor] = None,
            expert_gate_up_input_scale: Optional[Tensor] = None,
            expert_down_input_scale: Optional[Tensor] = None,
            mask_unselected_experts: bool = False,
            expert_affinities_eager: Optional[Tensor] = None,
            expert_affinities_scaling_mode=ExpertAffinityScaleMode.NO_SCALE,
            activation_fn="SiLU", output_dtype: Optional[torch.dtype] = None,
            gate_clamp_upper_limit: Optional[float] = None,
            gate_clamp_lower_limit: Optional[float] = None,
            up_clamp_upper_limit: Optional[float] = None,
            up_clamp_lower_limit: Optional[float] = None, output_in_sbuf: bool = False,
            is_all_expert_dynamic: bool = False, block_size: Optional[int] = None,
            input_dequant_scale: Optional[Tensor] = None,
            all_to_all_v_strategy=MoEAllToAllVStrategy.DISABLED) -> Tensor:
    """hidden_input bf16 [T, H]; expert_affinities [T, E] (global ids); expert_index [T, K].
    Weights packed or in the reference's Trainium MX layout (see moe_cte).  Returns [T, H]
    in output_dtype (bf16 by default)."""
    if member_name(all_to_all_v_strategy) != "DISABLED":
        raise NotImplementedError("all-to-all-v packed inputs need several GPUs")
    if hidden_input_scale is not None or expert_gate_up_input_scale is not None or \
            expert_down_input_scale is not None or input_dequant_scale is not None:
        raise NotImplementedError("FP8 activation quantization has no MI355X kernel")
    if expert_gate_up_weights.dtype not in (torch.uint8, torch.uint16, torch.int16):
        raise NotImplementedError(
            f"moe_tkg only supports MXFP4 weights, got {expert_gate_up_weights.dtype}")
    if hidden_input.dtype != torch.bfloat16:
        raise NotImplementedError("hidden_input must be bfloat16")
    if expert_affinities is None or expert_index is None:
        raise ValueError("expert_affinities and expert_index are required")
    ex = resolve_experts(expert_gate_up_weights, expert_gate_up_weights_scale,
                         expert_down_weights, expert_down_weights_scale, expert_gate_up_bias,
                         expert_down_bias)
    require_mxfp4(ex, "moe_tkg")
    idx = expert_index.to(torch.int64)
    val = torch.gather(expert_affinities.to(torch.float32), 1, idx)
    if rank_id is not None:
        idx = idx - ex.E * rank_id.reshape(-1)[0].to(idx.dtype)
    out = moe_tkg_raw(hidden_input, idx.to(torch.int32), val, ex, act_code(activation_fn),
                      _lib.clamps_array(gate_clamp_lower_limit, gate_clamp_upper_limit,
                                        up_clamp_lower_limit, up_clamp_upper_limit),
                      scale_code(expert_affinities_scaling_mode))
    if output_dtype is not None and output_dtype != out.dtype:
        out = out.to(output_dtype)
    return out
