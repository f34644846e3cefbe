"""MXFP4 MoE expert layer: the calls GPT-OSS makes into the operator API.

Counterpart of ``GptOssExperts`` (vllm_neuron/model/gpt_oss/model_mxfp4.py:841-1458
for the MXFP4 device path, model_bf16.py:1199-1413 for the CPU path) restricted to
the expert path at one GPU: the input is the already-normalized hidden state.
  * prefill (model_bf16.py:1282-1413): router (softmax over the top-k logits, fp32)
    -> build_blockwise_mapping (block 256) -> moe_cte (Swish, clamps gate <= limit,
    up in [-limit + 1, limit + 1], POST_SCALE, skip_token);
  * decode (model_bf16.py:1199-1252 through moe_block_tkg's expert part): router
    top-k -> moe_tkg in fp32 arithmetic.
Plain SwiGLU layers (no clamp, SiLU) use the same calls without clamps.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from .functional.moe.moe_blockwise import build_blockwise_mapping
from .functional.moe.moe_cte import moe_cte
from .functional.moe.moe_tkg import moe_tkg_raw
from .functional.moe.router import router_topk_raw
from .weights import MXFP4Experts

BLOCK_SIZE = 256  # model_mxfp4.py:937


class MXFP4MoE:
    def __init__(self, experts: MXFP4Experts, router_w: torch.Tensor,
                 router_b: Optional[torch.Tensor], top_k: int,
                 swiglu_limit: Optional[float] = 7.0, block_size: int = BLOCK_SIZE):
        self.w = experts
        self.router_w = router_w.contiguous()  # [E, H] bf16 or fp16
        self.router_b = None if router_b is None else router_b.contiguous()
        self._w_dt = _lib.dtype_code(self.router_w.dtype, "router weights",
                                     (torch.bfloat16, torch.float16))
        self._b_dt = (_lib.DT_BF16 if router_b is None
                      else _lib.dtype_code(router_b.dtype, "router bias"))
        self.top_k = top_k
        self.block_size = block_size
        self.limit = swiglu_limit
        if swiglu_limit is None:
            self.act = _lib.ACT_SILU
            self.clamp_args = (None, None, None, None)
        else:
            self.act = _lib.ACT_SWISH
            self.clamp_args = (None, swiglu_limit, -swiglu_limit + 1, swiglu_limit + 1)
        self._clamps = _lib.clamps_array(*self.clamp_args)
        self._ws = {}

    @property
    def E(self) -> int:
        return self.w.E

    def route(self, x: torch.Tensor):
        return router_topk_raw(x, self.router_w, self.top_k, self.router_b, _lib.ROUTER_SOFTMAX,
                               False, False, 0.0)

    def prefill(self, x: torch.Tensor, padding_mask: Optional[torch.Tensor] = None,
                output_dtype: torch.dtype = torch.bfloat16, stage_events=None):
        """Router, blockwise mapping and moe_cte in one library call (mxmoe_moe_prefill):
        the result of ``prefill_ops`` bit for bit, in four launches before the GEMMs
        instead of seven.  The workspace is cached per token count, so calls of one layer
        object belong on one stream.  stage_events: optional 5 torch.cuda.Event
        (enable_timing) recorded before the router, before the gate_up GEMM, after it,
        after the down GEMM and after the combine."""
        if output_dtype not in (torch.bfloat16, torch.float32):
            raise NotImplementedError("output_dtype must be bfloat16 or float32")
        w = self.w
        T, H = x.shape
        dev = _lib.require_cuda(x, w.gu_q)
        if x.dtype != torch.bfloat16 or H != w.H:
            raise ValueError(f"expected bf16 [T, {w.H}] hidden states")
        pm = None
        if padding_mask is not None:
            pm = padding_mask.reshape(-1).to(device=dev, dtype=torch.uint8).contiguous()
            if pm.numel() != T:
                raise ValueError(f"padding_mask has {pm.numel()} entries, expected {T}")
        L = _lib.lib()
        key = ("prefill", T)
        ws = self._ws.get(key)
        if ws is None:
            ws = _lib.workspace(L.mxmoe_moe_prefill_workspace_bytes(T, H, w.I, w.E, self.top_k,
                                                                    self.block_size), dev)
            self._ws[key] = ws
        x = x.contiguous()
        out = torch.empty(T, H, dtype=output_dtype, device=dev)
        rc = L.mxmoe_moe_prefill(
            x.data_ptr(), self.router_w.data_ptr(), self._w_dt, _lib.ptr(self.router_b),
            self._b_dt, _lib.ROUTER_SOFTMAX, 0, 0, 0.0, _lib.DT_F32, _lib.ptr(pm),
            w.gu_q.data_ptr(), w.gu_s.data_ptr(), w.dn_q.data_ptr(), w.dn_s.data_ptr(),
            _lib.WFMT_MXFP4, _lib.ptr(w.gu_bias), _lib.ptr(w.dn_bias), T, H, w.I, w.E, self.top_k,
            self.block_size, self.act, self._clamps, int(output_dtype == torch.float32),
            out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.event_array(stage_events),
            _lib.stream_handle(dev))
        _lib.check(rc, "mxmoe_moe_prefill")
        return out

    def prefill_ops(self, x: torch.Tensor, padding_mask: Optional[torch.Tensor] = None,
                    output_dtype: torch.dtype = torch.bfloat16, stage_events=None):
        """The prefill as the reference model calls the operators (model_bf16.py:1282-1413):
        router, build_blockwise_mapping, moe_cte, each its own library call.
        stage_events: optional 4 events around the moe_cte GEMMs and combine."""
        aff, _, _, _ = self.route(x)
        aff_m, tp2id, b2e, _ = build_blockwise_mapping(aff, self.E, self.top_k, self.block_size,
                                                       padding_mask=padding_mask)
        g_lo, g_hi, u_lo, u_hi = self.clamp_args
        w = self.w
        return moe_cte(x, aff_m, w.gu_q, w.dn_q, tp2id, b2e, self.block_size,
                       gate_and_up_proj_bias=w.gu_bias, down_proj_bias=w.dn_bias,
                       gate_up_proj_scale=w.gu_s, down_proj_scale=w.dn_s,
                       activation_function="Swish" if self.act == _lib.ACT_SWISH else "SiLU",
                       skip_token=True, expert_affinities_scaling_mode="POST_SCALE",
                       gate_clamp_upper_limit=g_hi, gate_clamp_lower_limit=g_lo,
                       up_clamp_upper_limit=u_hi, up_clamp_lower_limit=u_lo,
                       output_dtype=output_dtype, stage_events=stage_events)

    def decode(self, x: torch.Tensor, stage_events=None, logits_out=None, topk_idx_out=None):
        """Router + experts in one library call (mxmoe_moe_decode).  The workspace is
        cached per token count, so calls of one layer object belong on one stream.
        logits_out fp32 [T, E] / topk_idx_out int32 [T, k]: optional outputs of the
        front end (the logits and the experts it selected)."""
        w = self.w
        T, H = x.shape
        dev = _lib.require_cuda(x, w.gu_q)
        if x.dtype != torch.bfloat16 or H != w.H:
            raise ValueError(f"expected bf16 [T, {w.H}] hidden states")
        L = _lib.lib()
        ws = self._ws.get(T)
        if ws is None:
            ws = _lib.workspace(L.mxmoe_moe_decode_workspace_bytes(T, H, w.I, w.E, self.top_k), dev)
            self._ws[T] = ws
        x = x.contiguous()
        out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
        rc = L.mxmoe_moe_decode(
            x.data_ptr(), self.router_w.data_ptr(), self._w_dt, _lib.ptr(self.router_b),
            self._b_dt, _lib.ROUTER_SOFTMAX, 0, 0, 0.0, w.gu_q.data_ptr(), w.gu_s.data_ptr(),
            w.dn_q.data_ptr(), w.dn_s.data_ptr(), _lib.ptr(w.gu_bias), _lib.ptr(w.dn_bias), T, H,
            w.I, w.E, self.top_k, self.act, self._clamps, _lib.SCALE_POST, out.data_ptr(),
            _lib.ptr(logits_out), _lib.ptr(topk_idx_out), ws.data_ptr(), ws.numel(),
            _lib.event_array(stage_events), _lib.stream_handle(dev))
        _lib.check(rc, "mxmoe_moe_decode")
        return out
