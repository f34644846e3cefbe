"""Dense MLP with MX (MXFP4 or MXFP8) or bf16 weights on the MI355X kernels.

Mirrors vllm_neuron/functional/mlp.py:29-193 (signature, argument meaning, exception
types) for ``quantization_type`` MX and NONE.  The reference sends that case to the nkilib mlp
kernel (:114-175) and every case it cannot run to its torch flow ``_torch_mlp_impl``
(:313-418).  Here a dense MLP is the prefill expert path with one expert that every token
selects at affinity 1: the blockwise mapping of an all-ones [T, 1] affinity column (one
M-tile per 128 tokens, computed once per token count and device), then mxmoe_moe_cte with
E = 1, i.e. the grouped gate_up GEMM with fused dequant, bias, clamps and activation, and
the down GEMM with bias, with the torch flow's bf16 result of every op; the combine
multiplies by 1.0, which leaves the bf16 result unchanged.

Weights are this package's packed single-matrix layout (``weights.pack_mxfp4`` /
``weights.pack_mxfp8`` of the [out_features, in_features] matrix, i.e. the transpose of
the reference's ``x @ w`` operand): gate_w and up_w [I/16, 8H] (MXFP4) or [I/16, 16H]
(MXFP8) uint8 with scales [ceil(I/64), 2H]; down_w [H/16, 8I] or [H/16, 16I] with scales
[ceil(H/64), 2I].  gate and up fuse once per tensor version into an expert's gate_up
(``weights.fuse_gate_up``).  Biases: gate_b, up_b [1, I] or [I]; down_b [1, H] or [H], bf16.

With ``quantization_type=NONE`` the weights are the reference's bf16 operands (gate_w and
up_w [H, I], down_w [I, H], ``hidden @ w``): gate and up are stacked once per tensor
version into one expert's gate_up [1, H, 2, I] for the bf16 expert GEMMs.

Activations as the reference's ``_get_activation_fn`` (:261-286): SiLU and Swish are both
silu here (Swish is not GPT-OSS's 1.702 form in this operator), GELU the exact erf form.
The clamp limits, which the reference passes to its kernel only, are applied after the
biases as in moe_cte.  Raised as NotImplementedError: normalization, the fused
residual add, skip_gate, static input scales and GELU_Tanh_Approx; the FP8 types
(STATIC, ROW) and non-bf16 weights.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from .. import _lib
from ..enums import ActFnType, NormType, QuantizationType, member_name
from ..weights import fuse_gate_up
from .moe._cache import derived
from .moe._common import Experts, expert_shapes
from .moe.moe_blockwise import build_blockwise_mapping
from .moe.moe_cte import _cte_call

_BLOCK = 128
_MAPPINGS: dict = {}


def _act(act_fn) -> int:
    name = member_name(act_fn)
    if name in ("SiLU", "Swish"):
        return _lib.ACT_SILU
    if name == "GELU":
        return _lib.ACT_GELU
    raise NotImplementedError(f"mlp activation {name} has no MI355X kernel")


def _bias(b: Optional[Tensor], n: int, what: str) -> Optional[Tensor]:
    if b is None:
        return None
    if b.numel() != n or (b.dim() == 2 and b.shape[0] != 1) or b.dim() > 2:
        raise ValueError(f"{what} must be [1, {n}] or [{n}], got {tuple(b.shape)}")
    if b.dtype != torch.bfloat16:
        raise NotImplementedError(f"{what} must be bfloat16")
    return b.reshape(n)


def _experts(gate_w, gate_s, up_w, up_s, down_w, down_s, gate_b, up_b, down_b) -> Experts:
    for t, n in ((gate_w, "gate_w"), (up_w, "up_w"), (down_w, "down_w"), (gate_s, "gate_w_scale"),
                 (up_s, "up_w_scale"), (down_s, "down_w_scale")):
        if t.dtype != torch.uint8 or t.dim() != 2:
            raise ValueError(f"{n}: expected a packed uint8 [rows/16, bytes] tensor, got "
                             f"{t.dtype} {tuple(t.shape)}")

    def make():
        gu_q, gu_s = fuse_gate_up(gate_w, gate_s, up_w, up_s)
        gu_q, gu_s = gu_q.unsqueeze(0), gu_s.unsqueeze(0)
        dn_q, dn_s = down_w.contiguous().unsqueeze(0), down_s.contiguous().unsqueeze(0)
        E, H, I, fmt = expert_shapes(gu_q, gu_s, dn_q, dn_s)
        gb, ub, db = _bias(gate_b, I, "gate_b"), _bias(up_b, I, "up_b"), _bias(down_b, H, "down_b")
        gu_bias = dn_bias = None
        if gb is not None or ub is not None or db is not None:
            # A missing bias is a zero one: adding +0 to a bf16 result leaves it unchanged.
            z = lambda n: torch.zeros(n, dtype=torch.bfloat16, device=gate_w.device)  # noqa: E731
            gb = z(I) if gb is None else gb
            ub = z(I) if ub is None else ub
            gu_bias = torch.stack([gb, ub], 0).unsqueeze(0).contiguous()
            dn_bias = (z(H) if db is None else db).unsqueeze(0).contiguous()
        return Experts(gu_q, gu_s, dn_q, dn_s, gu_bias, dn_bias, E, H, I, fmt)

    return derived("mlp_experts",
                   (gate_w, gate_s, up_w, up_s, down_w, down_s, gate_b, up_b, down_b), make)


def _experts_bf16(gate_w, up_w, down_w, gate_b, up_b, down_b) -> Experts:
    """bf16 gate_w / up_w [H, I] and down_w [I, H] (the reference's ``x @ w`` operands) as
    one expert of the bf16 GEMMs: gate_up [1, H, 2, I] (a copy, kept per weight version),
    down [1, I, H] (a view)."""
    for t, n in ((gate_w, "gate_w"), (up_w, "up_w"), (down_w, "down_w")):
        if t.dtype != torch.bfloat16 or t.dim() != 2:
            raise NotImplementedError(f"{n}: quantization NONE takes bf16 [in, out] weights, got "
                                      f"{t.dtype} {tuple(t.shape)}")
    H, I = gate_w.shape
    if tuple(up_w.shape) != (H, I) or tuple(down_w.shape) != (I, H):
        raise ValueError(f"gate_w / up_w must be [H, I] and down_w [I, H], got "
                         f"{tuple(gate_w.shape)}, {tuple(up_w.shape)}, {tuple(down_w.shape)}")

    def make():
        gu = torch.stack([gate_w, up_w], 1).unsqueeze(0).contiguous()
        dn = down_w.contiguous().unsqueeze(0)
        gb, ub, db = _bias(gate_b, I, "gate_b"), _bias(up_b, I, "up_b"), _bias(down_b, H, "down_b")
        gu_bias = dn_bias = None
        if gb is not None or ub is not None or db is not None:
            z = lambda n: torch.zeros(n, dtype=torch.bfloat16, device=gate_w.device)  # noqa: E731
            gu_bias = torch.stack([z(I) if gb is None else gb, z(I) if ub is None else ub],
                                  0).unsqueeze(0).contiguous()
            dn_bias = (z(H) if db is None else db).unsqueeze(0).contiguous()
        return Experts(gu, None, dn, None, gu_bias, dn_bias, 1, H, I, _lib.WFMT_BF16)

    return derived("mlp_experts_bf16", (gate_w, up_w, down_w, gate_b, up_b, down_b), make)


def _identity_mapping(T: int, dev: torch.device):
    """(affinities [T, 1] = 1, token_position_to_id, block_to_expert, n_blocks) of T tokens
    all routed to expert 0, from the mapping kernel; kept per token count and device."""
    key = (T, dev)
    hit = _MAPPINGS.get(key)
    if hit is None:
        ones = torch.ones(T, 1, dtype=torch.float32, device=dev)
        aff_m, tp2id, b2e, _ = build_blockwise_mapping(ones, 1, 1, _BLOCK)
        hit = (aff_m.reshape(-1).contiguous(), tp2id.contiguous(), b2e.contiguous(),
               b2e.numel())
        # Tensors made during a graph capture live in the graph's pool: not kept.
        if not torch.cuda.is_current_stream_capturing():
            if len(_MAPPINGS) >= 16:
                _MAPPINGS.clear()
            _MAPPINGS[key] = hit
    return hit


def mlp(hidden: Tensor, gate_w: Tensor, up_w: Tensor, down_w: Tensor, eps: float = 1e-6,
        ln_w: Optional[Tensor] = None, skip_gate: bool = False, act_fn=ActFnType.SiLU,
        gate_b: Optional[Tensor] = None, up_b: Optional[Tensor] = None,
        down_b: Optional[Tensor] = None, norm_b: Optional[Tensor] = None,
        norm_type=NormType.NO_NORM, fused_add_tensor: Optional[Tensor] = None,
        store_fused_add_result: bool = False, quantization_type=QuantizationType.NONE,
        gate_w_scale: Optional[Tensor] = None, up_w_scale: Optional[Tensor] = None,
        down_w_scale: Optional[Tensor] = None, gate_up_in_scale: Optional[Tensor] = None,
        down_in_scale: Optional[Tensor] = None, quant_clipping_bound: float = 0.0,
        output_dtype: Optional[torch.dtype] = None,
        gate_clamp_upper_limit: Optional[float] = None,
        gate_clamp_lower_limit: Optional[float] = None,
        up_clamp_upper_limit: Optional[float] = None,
        up_clamp_lower_limit: Optional[float] = None, gate_up_w_layout=None) -> Tensor:
    """hidden [T, H] bf16 -> [T, H] in ``output_dtype`` (default: hidden's dtype; bf16 or
    float32, the latter being the bf16 result widened)."""
    q = member_name(quantization_type)
    if q not in ("MX", "NONE"):
        raise NotImplementedError(f"mlp with quantization_type {q} has no MI355X kernel (MX "
                                  "weights, or bf16 ones with NONE)")
    if member_name(norm_type) != "NO_NORM":
        raise NotImplementedError(f"mlp normalization {member_name(norm_type)} is not supported")
    if fused_add_tensor is not None or store_fused_add_result:
        raise NotImplementedError("mlp fused residual add is not supported")
    if skip_gate:
        raise NotImplementedError("mlp skip_gate is not supported")
    if gate_up_in_scale is not None or down_in_scale is not None:
        raise NotImplementedError("mlp static input scales are not supported")
    if gate_up_w_layout is not None:
        raise NotImplementedError("mlp gate_up_w_layout selects a Trainium layout")
    act = _act(act_fn)
    if q == "MX":
        if gate_w_scale is None or up_w_scale is None or down_w_scale is None:
            raise AssertionError("gate_w_scale, up_w_scale and down_w_scale must be provided "
                                 "for MX quantized compute")
        dev = _lib.require_cuda(hidden, gate_w, up_w, down_w, gate_w_scale, up_w_scale,
                                down_w_scale)
        ex = _experts(gate_w, gate_w_scale, up_w, up_w_scale, down_w, down_w_scale, gate_b, up_b,
                      down_b)
    else:
        if gate_w_scale is not None or up_w_scale is not None or down_w_scale is not None:
            raise NotImplementedError("weight scales belong to quantized weights; NONE takes "
                                      "bf16 weights without scales")
        dev = _lib.require_cuda(hidden, gate_w, up_w, down_w)
        ex = _experts_bf16(gate_w, up_w, down_w, gate_b, up_b, down_b)
    H = ex.H
    if hidden.dim() != 2 or hidden.shape[1] != H:
        raise ValueError(f"hidden must be [T, {H}], got {tuple(hidden.shape)}")
    if hidden.dtype != torch.bfloat16:
        raise NotImplementedError("hidden must be bfloat16")
    out_dt = hidden.dtype if output_dtype is None else output_dtype
    if out_dt not in (torch.bfloat16, torch.float32):
        raise NotImplementedError("output_dtype must be bfloat16 or float32")
    T = hidden.shape[0]
    out = torch.empty(T, H, dtype=out_dt, device=dev)
    if T == 0:
        return out
    aff, tp2id, b2e, n_blocks = _identity_mapping(T, dev)
    clamp_vals = (gate_clamp_lower_limit, gate_clamp_upper_limit, up_clamp_lower_limit,
                  up_clamp_upper_limit)
    _cte_call(hidden.contiguous(), aff, ex, None, tp2id, b2e, n_blocks, _BLOCK, T, act,
              clamp_vals, _lib.SCALE_POST, out)
    return out
