"""Prefill expert MLP (context encoding) on the MI355X kernel.

Mirrors vllm_neuron/functional/moe/moe_cte.py:37-420 (signature, argument
meaning, exception types).  The reference dispatches to nkilib moe_cte
(shard_on_block_mx for MXFP4, :650-732) or, on CPU and for non-MX weights, its
torch flow ``_torch_moe_impl`` (:448-581).  Here every call runs mxmoe_moe_cte:
the blockwise grouped gate_up GEMM with fused MXFP4 dequant, bias, clamps and
activation, the down GEMM with bias, and the affinity-weighted combine, with the
bf16 intermediate roundings of ``_torch_moe_impl``.  bf16 expert weights (the
shard_on_block operands of the bf16 model, model_bf16.py:1360-1391: gate_up [E, H, 2, I],
down [E, I, H], no scales) run the same schedule and epilogues on bf16 GEMMs; the MX
implementations (shard_on_block_mx, shard_on_i_mx, shard_on_i_mx_hybrid) require both
scales, as the reference asserts (:596-605).

Weights are the packed MXFP4 layout of vllm_neuron_amd.weights: gate_up_proj_weight
uint8 [E, 2I/16, 8H] with gate_up_proj_scale [E, ceil(2I/64), 2H]; down_proj_weight
[E, H/16, 8I] with down_proj_scale [E, ceil(H/64), 2I]; biases [E, 2, I] and [E, H].
The reference's own MX parameters (Trainium layout, model_mxfp4.py:957-1018, with the
tiled bias views of :1408-1420) are accepted as they are and converted once per tensor
version.

expert_affinities_scaling_mode (moe_cte.py:465-495, 518-579):
  * POST_SCALE: out = sum over the routed experts of y * affinity, fp32, ascending ids.
  * PRE_SCALE / PRE_SCALE_DELAYED: the affinity multiplies the hidden row before gate_up
    / the activation before down, and the output is the bf16 running sum over ALL E
    experts (:576-579).  The torch flow runs these modes with bf16 affinities (its
    einsums take one dtype), so the affinities are used rounded to bf16.  An expert a
    token does not route to adds its output for a zero input: the down bias under
    PRE_SCALE_DELAYED, and under PRE_SCALE y_e(0) = down(act(clamp(b_gate)) *
    clamp(b_up)) + b_down, computed once per weight version by the same kernels.
  * NO_SCALE: the torch flow adds every expert's full output for every token, routed or
    not, unscaled (its bf16 running sum over all E experts, as for PRE_SCALE_DELAYED with
    every affinity 1).  It runs as exactly that: a mapping that routes every token to every
    expert (T E slots: E times the routed work, the caller's mapping unused) and the
    PRE_SCALE_DELAYED kernels on affinities of 1, whose multiply is then exact.

Trainium tuning arguments (n_block_per_iter,
block_sharding_strategy, n_static_blocks, n_dynamic_blocks, checkpoint_activation,
skip_weight, ...) are accepted and have no effect; ``conditions`` is not needed
because empty blocks are detected from token_position_to_id.
"""

from __future__ import annotations

from typing import Any, Optional

import torch
from torch import Tensor

from ... import _lib
from ...enums import MoECTEImplementation, QuantizationType, member_name
from ._cache import derived
from ._common import act_code, is_bf16_weights, resolve_experts, scale_code

_MX_IMPLEMENTATIONS = ("shard_on_block_mx", "shard_on_i_mx", "shard_on_i_mx_hybrid")


def moe_cte(hidden_states: Tensor, expert_affinities_masked: Tensor, gate_up_proj_weight: Tensor,
            down_proj_weight: Tensor, token_position_to_id: Tensor, block_to_expert: Tensor,
            block_size: int, implementation=MoECTEImplementation.shard_on_block_mx,
            n_block_per_iter: int = 1, block_sharding_strategy=None, n_static_blocks: int = -1,
            n_dynamic_blocks: int = 55, checkpoint_activation: bool = False,
            expert_affinity_multiply_on_I: bool = False, num_static_block: Optional[int] = None,
            conditions: Optional[Tensor] = None, gate_and_up_proj_bias: Optional[Tensor] = None,
            down_proj_bias: Optional[Tensor] = None, gate_up_proj_scale: Optional[Tensor] = None,
            down_proj_scale: Optional[Tensor] = None,
            gate_up_activations_T: Optional[Tensor] = None,
            down_activations: Optional[Tensor] = None, activation_function="SiLU",
            skip_token: bool = False, skip_weight: bool = False, compute_dtype: Any = None,
            is_tensor_update_accumulating: bool = True,
            expert_affinities_scaling_mode="POST_SCALE",
            gate_clamp_upper_limit: Optional[float] = None,
            gate_clamp_lower_limit: Optional[float] = None,
            up_clamp_upper_limit: Optional[float] = None,
            up_clamp_lower_limit: Optional[float] = None,
            quantization_type=QuantizationType.NONE, gate_w_scale=None, up_w_scale=None,
            down_w_scale=None, gate_up_in_scale=None, down_in_scale=None,
            use_packed_scales: bool = False, output_dtype: torch.dtype = torch.bfloat16,
            stage_events=None) -> Tensor:
    """Returns the MoE output [T, H], T = expert_affinities_masked.shape[0] / E, in
    ``output_dtype``: bf16 (default, the device kernel's result) or float32 (the dtype
    of the reference torch flow, which promotes through the fp32 affinities).
    ``stage_events``: optional 4 torch.cuda.Event (enable_timing) recorded around the
    gate_up GEMM, the down GEMM and the combine."""
    if output_dtype not in (torch.bfloat16, torch.float32):
        raise NotImplementedError("output_dtype must be bfloat16 or float32")
    if member_name(quantization_type) == "STATIC_MX":
        raise NotImplementedError("STATIC_MX (FP8 weights) has no MI355X kernel")
    mode = scale_code(expert_affinities_scaling_mode, allow_no_scale=True, allow_pre=True)
    if gate_up_activations_T is not None or down_activations is not None:
        raise NotImplementedError("activation checkpoint buffers are not supported")
    bf16w = is_bf16_weights(gate_up_proj_weight)
    if member_name(implementation) in _MX_IMPLEMENTATIONS or not bf16w:
        # moe_cte.py:596-605: the MX implementations need both scales
        if gate_up_proj_scale is None or down_proj_scale is None:
            raise AssertionError(
                "gate_up_proj_scale and down_proj_scale must be provided for MX quantized "
                "compute")
        if bf16w:
            raise ValueError(f"{member_name(implementation)} takes packed MX weights, got "
                             f"{gate_up_proj_weight.dtype}")
    dev = _lib.require_cuda(hidden_states, expert_affinities_masked, gate_up_proj_weight,
                            down_proj_weight, token_position_to_id, block_to_expert)
    if (gate_and_up_proj_bias is None) != (down_proj_bias is None):
        raise ValueError("gate_and_up_proj_bias and down_proj_bias must both be provided or neither")
    ex = resolve_experts(gate_up_proj_weight, gate_up_proj_scale, down_proj_weight,
                         down_proj_scale, gate_and_up_proj_bias, down_proj_bias)
    E, H, I = ex.E, ex.H, ex.I
    if hidden_states.dim() != 2 or hidden_states.shape[1] != H:
        raise ValueError(f"hidden_states must be [T(+1), {H}], got {tuple(hidden_states.shape)}")
    if hidden_states.dtype != torch.bfloat16:
        raise NotImplementedError("hidden_states must be bfloat16")
    if block_size % 128 != 0:
        raise ValueError(f"block_size must be a multiple of 128, got {block_size}")
    if token_position_to_id.numel() % block_size != 0:
        raise ValueError("len(token_position_to_id) must be divisible by block_size")
    n_blocks = token_position_to_id.numel() // block_size
    if block_to_expert.numel() != n_blocks:
        raise ValueError(f"len(block_to_expert) must equal N = {n_blocks}")
    T = expert_affinities_masked.shape[0] // E
    if hidden_states.shape[0] < T:
        raise ValueError(f"hidden_states has {hidden_states.shape[0]} rows, need >= {T}")
    x = hidden_states.contiguous()
    aff = expert_affinities_masked.reshape(-1).to(torch.float32).contiguous()
    tp2id = token_position_to_id.reshape(-1).to(torch.int32).contiguous()
    b2e = block_to_expert.reshape(-1).to(torch.int32).contiguous()
    clamp_vals = (gate_clamp_lower_limit, gate_clamp_upper_limit, up_clamp_lower_limit,
                  up_clamp_upper_limit)
    act = act_code(activation_function)
    const = None
    if mode == _lib.SCALE_NO:
        return _no_scale(x, ex, T, block_size, act, clamp_vals, output_dtype, stage_events)
    if mode == _lib.SCALE_PRE_DELAYED:
        const = ex.dn_bias
    elif mode == _lib.SCALE_PRE and ex.gu_bias is not None:
        const = zero_input_outputs(ex, act, clamp_vals)
    out = torch.empty(T, H, dtype=output_dtype, device=dev)
    _cte_call(x, aff, ex, const, tp2id, b2e, n_blocks, block_size, T, act, clamp_vals, mode,
              out, stage_events)
    return out


def _no_scale(x, ex, T, block_size, act, clamp_vals, output_dtype, stage_events):
    """NO_SCALE (moe_cte.py:518-579 with no affinity applied): every expert on every token,
    the outputs added unscaled in expert order in bf16; the PRE_SCALE_DELAYED path over a
    mapping of all T E (token, expert) pairs with affinity 1."""
    from .moe_blockwise import build_blockwise_mapping

    E, H = ex.E, ex.H
    ones = torch.ones(T, E, dtype=torch.float32, device=x.device)
    aff_m, tp2id, b2e, _ = build_blockwise_mapping(ones, E, E, block_size)
    out = torch.empty(T, H, dtype=output_dtype, device=x.device)
    _cte_call(x, aff_m.reshape(-1), ex, ex.dn_bias, tp2id.reshape(-1), b2e.reshape(-1),
              b2e.numel(), block_size, T, act, clamp_vals, _lib.SCALE_PRE_DELAYED, out,
              stage_events)
    return out


def _cte_call(x, aff, ex, const, tp2id, b2e, n_blocks, block_size, T, act, clamp_vals, mode,
              out, stage_events=None):
    """mxmoe_moe_cte on prepared arguments; out [T, H] bf16 or fp32."""
    dev = x.device
    E, H, I = ex.E, ex.H, ex.I
    L = _lib.lib()
    ws = _lib.workspace(L.mxmoe_moe_cte_workspace_bytes(T, H, I, E, block_size, n_blocks, mode),
                        dev)
    clamps = _lib.clamps_array(*clamp_vals)
    gu_s = None if ex.gu_s is None else ex.gu_s.contiguous()
    dn_s = None if ex.dn_s is None else ex.dn_s.contiguous()
    rc = L.mxmoe_moe_cte(x.data_ptr(), aff.data_ptr(), ex.gu_q.contiguous().data_ptr(),
                         _lib.ptr(gu_s), ex.dn_q.contiguous().data_ptr(), _lib.ptr(dn_s), ex.fmt, _lib.ptr(ex.gu_bias),
                         _lib.ptr(ex.dn_bias), _lib.ptr(const), tp2id.data_ptr(), b2e.data_ptr(),
                         n_blocks, block_size, T, H, I, E, act, clamps, mode,
                         int(out.dtype == torch.float32), out.data_ptr(), ws.data_ptr(),
                         ws.numel(), _lib.event_array(stage_events), _lib.stream_handle(dev))
    _lib.check(rc, "mxmoe_moe_cte")


def zero_input_outputs(ex, act: int, clamp_vals) -> Tensor:
    """bf16 [E, H]: each expert's output for an all-zero hidden row (what a PRE_SCALE token
    that does not route to the expert adds, moe_cte.py:518-579).  Computed by the same
    kernels on E zero rows, row e routed to expert e alone with affinity 1 (an exact
    copy of y_e in the fp32 POST_SCALE combine), once per weight version and activation."""
    tag = f"zero_input_outputs:{act}:{clamp_vals}"

    def make():
        from .moe_blockwise import build_blockwise_mapping

        E, H = ex.E, ex.H
        dev = ex.gu_q.device
        aff = torch.eye(E, dtype=torch.float32, device=dev)
        aff_m, tp2id, b2e, _ = build_blockwise_mapping(aff, E, 1, 256)
        x0 = torch.zeros(E, H, dtype=torch.bfloat16, device=dev)
        y = torch.empty(E, H, dtype=torch.float32, device=dev)
        _cte_call(x0, aff_m.reshape(-1), ex, None, tp2id, b2e, b2e.numel(), 256, E, act,
                  clamp_vals, _lib.SCALE_POST, y)
        return y.to(torch.bfloat16)

    return derived(tag, (ex.gu_q, ex.gu_s, ex.dn_q, ex.dn_s, ex.gu_bias, ex.dn_bias), make)
