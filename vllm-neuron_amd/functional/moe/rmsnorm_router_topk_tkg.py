"""Fused RMSNorm + router top-k of the decode front end, on the MI355X kernels.

Mirrors vllm_neuron/functional/moe/rmsnorm_router_topk_tkg.py:33-45 (signature,
defaults, the validation of :123-174).  The reference runs an nkilib kernel or its
torch flow ``_torch_impl`` (:214-279); here one mxmoe_rmsnorm_router_topk call with the
torch flow's arithmetic:
  * inv_rms = rsqrt(sum(x^2 over all H) / hidden_actual + eps) in fp32; the norm
    x * inv_rms * gamma over every column, rounded to router_mm_dtype (the first output);
  * logits = norm . W (W cast to router_mm_dtype, fp32 accumulation) + the bias cast to
    router_mm_dtype, in fp32;
  * top-k on the fp32 logits, the activation over the k selected values (fp32), scattered
    into bf16 affinities (zeros elsewhere); expert_index int32.

quantization_type MX (the fused MXFP8 quantization of the norm, :282-341) follows
nkilib's quantize_mx_golden, which the reference does not contain: it raises
NotImplementedError, as do router_mm_dtype float32 and the SIGMOID/SOFTMAX-free
activations.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from ... import _lib
from ...enums import QuantizationType, RouterActFnType, member_name
from ._cache import transposed_rows


def _validate_inputs(hidden_states, gamma, router_weights, router_bias, top_k, hidden_actual,
                     quantization_type, router_act_fn) -> None:
    """rmsnorm_router_topk_tkg.py:123-174 (same conditions, AssertionError as there)."""
    fn = member_name(router_act_fn)
    assert fn in ("SIGMOID", "SOFTMAX"), f"router_act_fn must be SIGMOID or SOFTMAX, got {fn}"
    assert hidden_states.ndim == 3, (
        f"hidden_states must be [B, S, H], got shape {tuple(hidden_states.shape)}")
    B, S, H = hidden_states.shape
    assert tuple(gamma.shape) in ((1, H), (H,)), (
        f"gamma must be [1, {H}] or [{H}], got shape {tuple(gamma.shape)}")
    assert router_weights.ndim == 2 and router_weights.shape[0] == H, (
        f"router_weights must be [H={H}, E], got shape {tuple(router_weights.shape)}")
    E = router_weights.shape[1]
    if router_bias is not None:
        assert tuple(router_bias.shape) == (1, E), (
            f"router_bias must be [1, {E}], got shape {tuple(router_bias.shape)}")
    assert 1 <= top_k <= E, f"top_k must be in [1, E={E}], got top_k={top_k}"
    assert H % 256 == 0, f"H must be divisible by 256, got H={H}"
    if hidden_actual is not None:
        assert 0 < hidden_actual <= H, (
            f"hidden_actual must be in (0, H={H}], got hidden_actual={hidden_actual}")
    qt = member_name(quantization_type)
    assert qt in ("NONE", "MX"), f"quantization_type must be NONE or MX, got {qt}"
    if qt == "MX":
        assert H % 512 == 0, f"H must be divisible by 512 for MX quantization, got H={H}"


def rmsnorm_router_topk_tkg(hidden_states: Tensor, gamma: Tensor, router_weights: Tensor,
                            router_bias: Optional[Tensor] = None, eps: float = 1e-6,
                            top_k: int = 1, hidden_actual: Optional[int] = None,
                            quantization_type=QuantizationType.NONE,
                            router_mm_dtype: torch.dtype = torch.bfloat16,
                            router_act_fn=RouterActFnType.SIGMOID
                            ) -> Tuple[Tensor, Tensor, Tensor]:
    """hidden_states bf16 [B, S, H]; gamma [1, H] or [H]; router_weights [H, E] (bf16 or
    fp16); router_bias [1, E].  Returns (norm [T, H] in router_mm_dtype, expert_index
    int32 [T, k], expert_affinities bf16 [T, E])."""
    _validate_inputs(hidden_states, gamma, router_weights, router_bias, top_k, hidden_actual,
                     quantization_type, router_act_fn)
    if member_name(quantization_type) == "MX":
        raise NotImplementedError(
            "quantization_type=MX (fused MXFP8 quantization) has no MI355X kernel")
    mm = _lib.dtype_code(router_mm_dtype, "router_mm_dtype", (torch.float16, torch.bfloat16))
    if hidden_states.dtype != torch.bfloat16:
        raise NotImplementedError(f"hidden_states must be bfloat16, got {hidden_states.dtype}")
    dev = _lib.require_cuda(hidden_states, gamma, router_weights, router_bias)
    B, S, H = hidden_states.shape
    T = B * S
    E = router_weights.shape[1]
    x = hidden_states.reshape(T, H).contiguous()
    g = gamma.reshape(-1).to(torch.float32).contiguous()
    w_eh = transposed_rows(router_weights)
    wdt = _lib.dtype_code(w_eh.dtype, "router_weights", (torch.bfloat16, torch.float16))
    bias = None if router_bias is None else router_bias.reshape(-1).contiguous()
    bdt = _lib.DT_BF16 if bias is None else _lib.dtype_code(bias.dtype, "router_bias")
    act = _lib.ROUTER_SOFTMAX if member_name(router_act_fn) == "SOFTMAX" else _lib.ROUTER_SIGMOID
    norm = torch.empty(T, H, dtype=router_mm_dtype, device=dev)
    idx = torch.empty(T, top_k, dtype=torch.int32, device=dev)
    aff = torch.empty(T, E, dtype=torch.bfloat16, device=dev)
    L = _lib.lib()
    ws = _lib.workspace(L.mxmoe_rmsnorm_router_topk_workspace_bytes(T, E, top_k), dev)
    ha = H if hidden_actual is None else int(hidden_actual)
    rc = L.mxmoe_rmsnorm_router_topk(x.data_ptr(), g.data_ptr(), ha, float(eps), w_eh.data_ptr(),
                                     wdt, _lib.ptr(bias), bdt, T, H, E, top_k, act, mm,
                                     norm.data_ptr(), idx.data_ptr(), aff.data_ptr(),
                                     ws.data_ptr(), ws.numel(), _lib.stream_handle(dev))
    _lib.check(rc, "mxmoe_rmsnorm_router_topk")
    return norm, idx, aff
