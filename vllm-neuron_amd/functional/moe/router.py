"""Router: linear -> top-k -> activation -> scatter, on the MI355X kernel.

Mirrors vllm_neuron/functional/moe/router.py:71-297 (same signature, argument
meaning, validation and exception types, _validate_router_inputs :601-677).  The
reference dispatches to nkilib router_topk (:690-796) or its torch flow
(:383-565); here every supported call runs mxmoe_router_topk (after mxmoe_rmsnorm when
gamma is given) and anything the kernels do not cover raises NotImplementedError
(there is no CPU path).  computation_dtype float32, float16 and bfloat16 follow the
torch flow's arithmetic in that dtype (router.py:414-440): operands cast to it, fp32
sums of the products, one rounding per tensor op; the GPT-OSS MXFP4 model passes
float16 with float16 router weights (model_mxfp4.py:950-955, :1337-1344).

Computation orders: PRENORM_LINEAR_TOPK_ACT_SCATTER and
PRENORM_LINEAR_ACT_TOPK_RENORM_SCATTER run as in the reference.
PRENORM_LINEAR_TOPK_SCATTER_ACT scatters the k logits into -inf and applies the
activation to the whole row; softmax and sigmoid of -inf are 0, so it selects and
weights exactly like PRENORM_LINEAR_TOPK_ACT_SCATTER and runs on that path.
"""

from __future__ import annotations

from typing import Callable, Optional, Tuple, Union

import torch
from torch import Tensor

from ... import _lib
from ...enums import RouterComputationOrder
from ._cache import transposed_rows


def _validate_router_inputs(hidden_states, router_weights, top_k, router_bias, gamma,
                            computation_dtype, router_computation_order,
                            transposed_hidden_states):
    """router.py:601-677."""
    if hidden_states.dim() != 2:
        raise ValueError(f"Expected hidden_states to be 2D [T, H], got shape {hidden_states.shape}")
    if router_weights.dim() != 2:
        raise ValueError(f"Expected router_weights to be 2D [H, E], got shape {router_weights.shape}")
    if transposed_hidden_states:
        H, T = hidden_states.shape
    else:
        T, H = hidden_states.shape
    H_w, E = router_weights.shape
    if H != H_w:
        raise ValueError(f"Hidden dimension mismatch: hidden_states has {H}, router_weights has {H_w}")
    if router_bias is not None and tuple(router_bias.shape) != (E,):
        raise ValueError(f"Expected router_bias shape [E], got {router_bias.shape}")
    if gamma is not None and tuple(gamma.shape) != (H,):
        raise ValueError(f"Expected gamma shape [H], got {gamma.shape}")
    if top_k < 1 or top_k > E:
        raise ValueError(f"top_k must be between 1 and {E}, got {top_k}")
    if computation_dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ValueError(f"computation_dtype must be float32/float16/bfloat16, got {computation_dtype}")
    if not isinstance(router_computation_order, RouterComputationOrder) and \
            getattr(router_computation_order, "name", None) not in RouterComputationOrder.__members__:
        raise ValueError("router_computation_order must be a RouterComputationOrder enum, "
                         f"got {type(router_computation_order)}")


def _act_code(activation) -> int:
    if isinstance(activation, str):
        if activation == "softmax":
            return _lib.ROUTER_SOFTMAX
        if activation == "sigmoid":
            return _lib.ROUTER_SIGMOID
        raise ValueError(f"Unsupported activation function: {activation}. Use 'softmax' or 'sigmoid'.")
    if callable(activation):
        raise NotImplementedError("callable router activations have no MI355X kernel")
    raise ValueError("Activation must be either a string ('softmax' or 'sigmoid') or a callable "
                     f"function. Got: {type(activation)}")


def router_topk_raw(x: Tensor, w_eh: Tensor, top_k: int, bias: Optional[Tensor], act: int,
                    act_before_topk: bool, renorm: bool, renorm_eps: float = 0.0,
                    compute_dtype: torch.dtype = torch.float32):
    """Kernel call.  x bf16 (or fp16 with compute_dtype fp16) [T, H]; w_eh bf16/fp16 [E, H];
    bias [E] (fp32, fp16 or bf16) or None.  Returns (affinities [T, E], logits [T, E],
    topk_idx int32 [T, k], topk_val fp32 [T, k]); affinities and logits in fp32 holding
    values of compute_dtype."""
    dev = _lib.require_cuda(x, w_eh, bias)
    T, H = x.shape
    E = w_eh.shape[0]
    xdt = _lib.dtype_code(x.dtype, "hidden_states", (torch.bfloat16, torch.float16))
    wdt = _lib.dtype_code(w_eh.dtype, "router_weights", (torch.bfloat16, torch.float16))
    bdt = _lib.DT_BF16 if bias is None else _lib.dtype_code(bias.dtype, "router_bias")
    cdt = _lib.dtype_code(compute_dtype, "computation_dtype")
    x = x.contiguous()
    w_eh = w_eh.contiguous()
    if bias is not None:
        bias = bias.contiguous()
    aff = torch.empty(T, E, dtype=torch.float32, device=dev)
    logits = torch.empty(T, E, dtype=torch.float32, device=dev)
    idx = torch.empty(T, top_k, dtype=torch.int32, device=dev)
    val = torch.empty(T, top_k, dtype=torch.float32, device=dev)
    L = _lib.lib()
    rc = L.mxmoe_router_topk(x.data_ptr(), xdt, w_eh.data_ptr(), wdt, _lib.ptr(bias), bdt, T, H,
                             E, top_k, act, int(act_before_topk), int(renorm), float(renorm_eps),
                             cdt, logits.data_ptr(), aff.data_ptr(), idx.data_ptr(),
                             val.data_ptr(), None, 0, _lib.stream_handle(dev))
    _lib.check(rc, "mxmoe_router_topk")
    return aff, logits, idx, val


def rms_norm(x: Tensor, gamma: Tensor, eps: float, hidden_actual: Optional[int] = None,
             all_cols: bool = True, out_dtype: Optional[torch.dtype] = None) -> Tensor:
    """mxmoe_rmsnorm: bf16 [T, H] -> [T, H] in out_dtype (bf16 or fp16; default bf16).
    all_cols: mean square over all H columns divided by hidden_actual (router.py:680-687
    with hidden_actual = H, rmsnorm_router_topk_tkg.py:249-257); otherwise over the
    first hidden_actual columns with the others zeroed (moe_block_tkg.py:134-150)."""
    dev = _lib.require_cuda(x, gamma)
    if x.dtype != torch.bfloat16:
        raise NotImplementedError(f"the MI355X RMSNorm takes bfloat16 rows, got {x.dtype}")
    T, H = x.shape
    ha = H if hidden_actual is None else int(hidden_actual)
    g = gamma.reshape(-1).to(torch.float32).contiguous()
    if g.numel() != H:
        raise ValueError(f"gamma has {g.numel()} elements, expected {H}")
    odt = torch.bfloat16 if out_dtype is None else out_dtype
    code = _lib.dtype_code(odt, "RMSNorm output", (torch.bfloat16, torch.float16))
    out = torch.empty(T, H, dtype=odt, device=dev)
    rc = _lib.lib().mxmoe_rmsnorm(x.contiguous().data_ptr(), g.data_ptr(), T, H, ha,
                                  int(all_cols), float(eps), code, out.data_ptr(),
                                  _lib.stream_handle(dev))
    _lib.check(rc, "mxmoe_rmsnorm")
    return out


def router(hidden_states: Tensor, router_weights: Tensor, top_k: int,
           router_bias: Optional[Tensor] = None,
           activation: Union[str, Callable[[Tensor], Tensor]] = "softmax",
           return_logits: bool = False, gamma: Optional[Tensor] = None, eps: float = 1e-6,
           computation_dtype: torch.dtype = torch.float32,
           router_computation_order: RouterComputationOrder =
           RouterComputationOrder.PRENORM_LINEAR_TOPK_ACT_SCATTER,
           shard_on_tokens: Optional[bool] = None, transposed_hidden_states: bool = False,
           x_sb_layout: Optional[int] = None, use_column_tiling: Optional[bool] = None,
           use_indirect_dma_scatter: Optional[bool] = None,
           use_PE_broadcast_w_bias: Optional[bool] = None) -> Union[Tensor, Tuple[Tensor, Tensor]]:
    """Router API (router.py:71-297).  hidden_states bf16 [T, H] (or [H, T] when
    transposed), router_weights bf16/fp16 [H, E] (typically ``W.T`` of a [E, H]
    parameter), router_bias [E], gamma [H] (optional RMSNorm before the router,
    router.py:680-687).  Returns affinities [T, E] (+ logits [T, E]) in
    ``computation_dtype``, computed as the torch flow computes them in that dtype
    (router.py:414-440).

    Kernel-only tuning arguments of the reference (shard_on_tokens, x_sb_layout,
    use_column_tiling, use_indirect_dma_scatter, use_PE_broadcast_w_bias) are accepted
    and have no effect."""
    _validate_router_inputs(hidden_states, router_weights, top_k, router_bias, gamma,
                            computation_dtype, router_computation_order,
                            transposed_hidden_states)
    act = _act_code(activation)
    x = hidden_states.t() if transposed_hidden_states else hidden_states
    if x.dtype != torch.bfloat16:
        raise NotImplementedError(
            f"the MI355X router takes bfloat16 hidden_states, got {x.dtype}")
    if gamma is not None:
        x = rms_norm(x, gamma, eps)
    w_eh = transposed_rows(router_weights)
    name = getattr(router_computation_order, "name", "")
    act_first = name == "PRENORM_LINEAR_ACT_TOPK_RENORM_SCATTER"
    aff, logits, _, _ = router_topk_raw(x, w_eh, top_k, router_bias, act, act_first, act_first,
                                        0.0, computation_dtype)
    if computation_dtype != torch.float32:  # the values already are of that dtype
        aff = aff.to(computation_dtype)
        logits = logits.to(computation_dtype)
    return (aff, logits) if return_logits else aff
