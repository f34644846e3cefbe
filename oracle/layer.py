"""Oracle: the GPT-OSS expert layer as the reference's CPU mode runs it.

Test infrastructure only (see ``oracle/__init__.py``).

Follows vllm_neuron/model/gpt_oss/model_bf16.py:
  * ``RefLayer.__init__``  <- the bf16 parameters the MXFP4 checkpoint is loaded into
    (weight_loaders_bf16.py:319-488): gate_up [E, H, 2I] = [gate | up], gate_up bias
    [E, 2I] = [gate | up + 1], down [E, I, H], down bias [E, H]; router weight [E, H]
  * ``RefLayer.prefill``   <- ``forward_prefill`` (:1282-1413) minus the RMSNorm: router
    (softmax, fp32, :1297-1305) -> build_blockwise_mapping (block 256, :1341-1357) ->
    moe_cte torch flow (:1359-1386: Swish, gate <= limit, up in [-limit+1, limit+1],
    POST_SCALE)
  * ``RefLayer.decode``    <- ``_run_moe_block_tkg`` (:1199-1252) expert part with the
    router of the same call (router_pre_norm=False, softmax), fp32 arithmetic, bf16 out
Plain-SwiGLU layers (no limit) use SiLU, no clamps, no biases.

The ``routed`` variants compute only the selected experts (and optionally a subset of
tokens) and are pinned against the dense ones in tests/test_oracle_moe.py.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import blockwise, moe_block_tkg, moe_cte, mxfp4, router


class LazyExperts:
    """Per-expert dequantized weights made on first use (a few kept): the indexing the
    routed forms use (``w[e]``, ``w[e, :, 0, :]``) on a layer too large to dequantize at
    once.  ``kind`` "gate_up" gives [H, 2, I] per expert, "down" [I, H]."""

    def __init__(self, kind, blocks, scales, E, H, I, keep=4):
        self.kind, self.blocks, self.scales = kind, blocks, scales
        self.shape = (E, H, 2, I) if kind == "gate_up" else (E, I, H)
        self.H, self.I, self.keep = H, I, keep
        self._cache = {}

    def _get(self, e: int) -> torch.Tensor:
        w = self._cache.get(e)
        if w is None:
            if self.kind == "gate_up":
                w = mxfp4.gate_up_from_checkpoint(self.blocks[e:e + 1], self.scales[e:e + 1])
                w = w.reshape(self.H, 2, self.I)
            else:
                w = mxfp4.down_from_checkpoint(self.blocks[e:e + 1], self.scales[e:e + 1])[0]
            if len(self._cache) >= self.keep:
                self._cache.pop(next(iter(self._cache)))
            self._cache[e] = w
        return w

    def __getitem__(self, idx):
        if isinstance(idx, tuple):
            return self._get(int(idx[0]))[idx[1:]]
        return self._get(int(idx))


class RefLayer:
    def __init__(self, lt, lazy: bool = False):
        """``lt``: a LayerTensors-like object with checkpoint-layout CPU tensors.  lazy:
        dequantize experts one at a time when a routed form needs them (the dense flows
        then are unavailable)."""
        self.shape = lt.shape
        self.K = lt.shape.K
        self.limit = lt.shape.swiglu_limit
        self.lazy = lazy
        if lazy:
            E, twoI, Gh, _ = lt.gate_up_blocks.shape
            H, I = Gh * 32, twoI // 2
            self.gate_up = None
            self.down = LazyExperts("down", lt.down_blocks, lt.down_scales, E, H, I)
            self._gu_lazy = LazyExperts("gate_up", lt.gate_up_blocks, lt.gate_up_scales, E, H, I)
            self.E, self.H, self.I = E, H, I
        else:
            self.gate_up = mxfp4.gate_up_from_checkpoint(lt.gate_up_blocks, lt.gate_up_scales)
            self.down = mxfp4.down_from_checkpoint(lt.down_blocks, lt.down_scales)
            self.E, self.H, twoI = self.gate_up.shape
            self.I = twoI // 2
        self.gu_bias = (None if lt.gate_up_bias is None
                        else mxfp4.gate_up_bias_from_checkpoint(lt.gate_up_bias))
        self.dn_bias = lt.down_bias
        self.router_w = lt.router_w
        self.router_b = lt.router_b
        self._set_activation()

    def _set_activation(self):
        """GPT-OSS's call (model_bf16.py:1359-1386): Swish, gate <= limit, up in
        [-limit + 1, limit + 1]; plain SwiGLU (no limit): SiLU, no clamps."""
        if self.limit is None:
            self.act = moe_cte.SILU
            self.clamps = dict(gate_clamp_upper_limit=None, gate_clamp_lower_limit=None,
                               up_clamp_upper_limit=None, up_clamp_lower_limit=None)
        else:
            self.act = moe_cte.SWISH
            self.clamps = dict(gate_clamp_upper_limit=self.limit, gate_clamp_lower_limit=None,
                               up_clamp_upper_limit=self.limit + 1,
                               up_clamp_lower_limit=-self.limit + 1)

    @classmethod
    def from_dense(cls, gate_up, down, gu_bias, dn_bias, router_w, router_b, top_k,
                   swiglu_limit):
        """A layer from bf16 parameters as the reference's CPU model holds them
        (weight_loaders_bf16.py:319-488 outputs): gate_up [E, H, 2I] = [gate | up], down
        [E, I, H], gate_up bias [E, 2I] (up half with its +1), down bias [E, H], router
        weight [E, H]."""
        self = cls.__new__(cls)
        self.gate_up, self.down = gate_up, down
        self.E, self.H, twoI = gate_up.shape
        self.I = twoI // 2
        self.gu_bias, self.dn_bias = gu_bias, dn_bias
        self.router_w, self.router_b = router_w, router_b
        self.K, self.limit, self.lazy = top_k, swiglu_limit, False
        self.shape = None
        self._set_activation()
        return self

    # ---- routing (router.py torch flow, fp32)
    def route(self, x: torch.Tensor):
        return router.topk_act_scatter(x.to(torch.float32), self.router_w.T, self.K,
                                       self.router_b, "softmax", None, 1e-6, torch.float32)

    # ---- prefill
    def _gu4(self):
        """gate_up as [E, H, 2, I] (or its lazy per-expert form)."""
        if self.lazy:
            return self._gu_lazy
        return self.gate_up.reshape(self.E, self.H, 2, self.I)

    def _cte_args(self):
        gu = self._gu4()
        gb = None if self.gu_bias is None else self.gu_bias.reshape(self.E, 2, self.I)
        db = None if self.dn_bias is None else self.dn_bias.unsqueeze(1)
        return gu, gb, db

    def prefill(self, x: torch.Tensor, aff: Optional[torch.Tensor] = None):
        """Dense reference flow; returns (out fp32 [T, H], affinities [T, E])."""
        if aff is None:
            aff, _ = self.route(x)
        aff_m, _, _, _ = blockwise.build_blockwise_mapping(aff, self.E, self.K, 256)
        gu, gb, db = self._cte_args()
        out = moe_cte.torch_moe_impl(x, aff_m, gu, self.down, gb, db, activation_function=self.act,
                                     expert_affinities_scaling_mode=moe_cte.POST_SCALE,
                                     **self.clamps)
        return out, aff

    def prefill_routed(self, x: torch.Tensor, aff: torch.Tensor, token_rows=None):
        gu, gb, db = self._cte_args()
        return moe_cte.torch_moe_impl_routed(x, aff.reshape(-1, 1), gu, self.down, gb, db,
                                             activation_function=self.act,
                                             expert_affinities_scaling_mode=moe_cte.POST_SCALE,
                                             token_rows=token_rows, **self.clamps)

    # ---- decode
    def decode(self, x: torch.Tensor, aff: Optional[torch.Tensor] = None):
        """Dense fp32 expert flow; returns (out bf16 [T, H], affinities [T, E])."""
        if aff is None:
            aff, _ = self.route(x)
        gu = self.gate_up.reshape(self.E, self.H, 2, self.I)
        gb = None if self.gu_bias is None else self.gu_bias.reshape(self.E, 2, self.I)
        x32 = x.to(torch.float32)
        g_u = torch.einsum("th,ehi->eti", x32, gu.reshape(self.E, self.H, 2 * self.I).float())
        if gb is not None:
            g_u = g_u + gb.reshape(self.E, 2 * self.I).unsqueeze(1).float()
        gate, up = torch.chunk(g_u, 2, dim=-1)
        c = self.clamps
        if c["gate_clamp_lower_limit"] is not None or c["gate_clamp_upper_limit"] is not None:
            gate = gate.clamp(min=c["gate_clamp_lower_limit"], max=c["gate_clamp_upper_limit"])
        if c["up_clamp_lower_limit"] is not None or c["up_clamp_upper_limit"] is not None:
            up = up.clamp(min=c["up_clamp_lower_limit"], max=c["up_clamp_upper_limit"])
        inter = up * moe_block_tkg._act(gate, self.act)
        nxt = torch.einsum("eti,eih->eth", inter, self.down.float())
        if self.dn_bias is not None:
            nxt = nxt + self.dn_bias.unsqueeze(1).float()
        out = torch.zeros(x.shape[0], self.H, dtype=torch.float32)
        for e in range(self.E):
            out = out + nxt[e] * aff[:, e:e + 1]
        return out.to(x.dtype), aff

    def decode_routed(self, x: torch.Tensor, aff: torch.Tensor):
        gu = self._gu4()
        gb = None if self.gu_bias is None else self.gu_bias.reshape(self.E, 2, self.I)
        return moe_block_tkg.expert_mlp_fp32_routed(
            x, aff, gu, self.down, gb, self.dn_bias, hidden_act_fn=self.act,
            scale_mode="POST_SCALE", out_dtype=x.dtype, **self.clamps)
