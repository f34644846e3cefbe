"""Oracle: decode MoE block (``moe_block_tkg`` torch fallback), fp32 expert math.

Test infrastructure only (see ``oracle/__init__.py``).

Follows vllm_neuron/functional/moe/moe_block_tkg.py:56-302
(``_torch_moe_block_tkg_impl``): RMSNorm over the unpadded hidden size with the
result cast back to the input dtype (:134-150), fp32 router logits (:152-162),
top-k then activation (router_pre_norm=False, :185-204) or activation then top-k
(:166-183), optional L1 renorm with +1e-20 (:180-183, :199-202), local affinities
(:206-221), fp32 gate/up einsum over all local experts (:223-238), clamps
(:243-248), activation (:250-263), fp32 down einsum and bias (:265-276), and the
weighted sum over experts in ascending order (:278-295), cast to the input dtype.

``expert_mlp_fp32_routed`` is the expert part (:223-297) evaluated only on the
selected experts, from given affinities; its agreement with the dense form is
pinned in tests/test_oracle_moe.py on small shapes.
"""

from __future__ import annotations

from typing import Optional

import torch

from .moe_cte import SILU, GELU, SWISH, _name

SOFTMAX = "SOFTMAX"
SIGMOID = "SIGMOID"
NO_SCALE = "NO_SCALE"


def _act(g, act):
    act = _name(act)
    if act == SILU:
        return torch.nn.functional.silu(g)
    if act == GELU:
        return torch.nn.functional.gelu(g)
    if act == SWISH:
        return g * torch.sigmoid(g * 1.702)
    raise NotImplementedError(f"Activation function {act} is not supported")


def rmsnorm_router(inp, gamma, router_weights, router_bias, eps, top_k, router_act_fn,
                   router_pre_norm, norm_topk_prob, hidden_actual=None):
    """moe_block_tkg.py:120-204. Returns (x_norm [T,H] in inp dtype, logits fp32 [T,E],
    top values fp32 [T,k], top indices int64 [T,k])."""
    if inp.dim() == 3:
        inp = inp.reshape(-1, inp.shape[-1])
    H = inp.shape[-1]
    dtype = inp.dtype
    ha = H if hidden_actual is None else hidden_actual
    x32 = inp.to(torch.float32)
    xn = x32.clone()
    var = x32[..., :ha].pow(2).mean(-1, keepdim=True)
    xn[..., :ha] = xn[..., :ha] * torch.rsqrt(var + eps)
    g = gamma.squeeze(0) if gamma.dim() == 2 else gamma
    xn = (g * xn).to(dtype)
    xn[..., ha:] = 0.0
    logits = torch.matmul(xn.to(torch.float32), router_weights.to(torch.float32))
    if router_bias is not None:
        b = router_bias.to(torch.float32)
        if b.dim() == 2:
            b = b.squeeze(0)
        logits = logits + b
    fn = _name(router_act_fn)
    if router_pre_norm:
        if fn == SOFTMAX:
            act = torch.nn.functional.softmax(logits, dim=-1, dtype=torch.float32)
        elif fn == SIGMOID:
            act = torch.sigmoid(logits)
        else:
            raise NotImplementedError(fn)
        top, idx = torch.topk(act, top_k, dim=-1)
        if norm_topk_prob:
            top = top / (top.sum(dim=-1, keepdim=True) + 1e-20)
    else:
        top, idx = torch.topk(logits, top_k, dim=-1)
        if fn == SOFTMAX:
            top = torch.nn.functional.softmax(top, dim=-1, dtype=torch.float32)
        elif fn == SIGMOID:
            top = torch.sigmoid(top)
        else:
            raise NotImplementedError(fn)
        if norm_topk_prob:
            top = top / (top.sum(dim=-1, keepdim=True) + 1e-20)
    return xn, logits, top, idx


def torch_moe_block_tkg_impl(inp, gamma, router_weights, expert_gate_up_weights,
                             expert_down_weights, router_bias=None, expert_gate_up_bias=None,
                             expert_down_bias=None, eps=1e-6, top_k=1, router_act_fn=SIGMOID,
                             router_pre_norm=True, norm_topk_prob=False,
                             expert_affinities_scaling_mode=NO_SCALE, hidden_act_fn=SILU,
                             gate_clamp_upper_limit=None, gate_clamp_lower_limit=None,
                             up_clamp_upper_limit=None, up_clamp_lower_limit=None,
                             hidden_actual=None, skip_router_logits=False, rank_id=None):
    """moe_block_tkg.py:56-302 (dense over all local experts)."""
    if inp.dim() == 3:
        inp = inp.reshape(-1, inp.shape[-1])
    T, H = inp.shape
    dtype = inp.dtype
    E_L, _, _, I = expert_gate_up_weights.shape
    E_g = router_weights.shape[1]
    xn, logits, top, idx = rmsnorm_router(inp, gamma, router_weights, router_bias, eps, top_k,
                                          router_act_fn, router_pre_norm, norm_topk_prob,
                                          hidden_actual)
    if E_L < E_g and rank_id is not None:
        start = E_L * int(rank_id.reshape(-1)[0])
        full = torch.zeros(T, E_g, dtype=torch.float32).scatter_(1, idx, top)
        aff = full[:, start:start + E_L]
    else:
        aff = torch.zeros(T, E_L, dtype=torch.float32).scatter_(1, idx, top)
    gu = torch.einsum("th,ehi->eti", xn.to(torch.float32),
                      expert_gate_up_weights.reshape(E_L, H, 2 * I).to(torch.float32))
    if expert_gate_up_bias is not None:
        gu = gu + expert_gate_up_bias.reshape(E_L, 2 * I).unsqueeze(1).to(torch.float32)
    gate, up = torch.chunk(gu, chunks=2, dim=-1)
    if gate_clamp_lower_limit is not None or gate_clamp_upper_limit is not None:
        gate = gate.clamp(min=gate_clamp_lower_limit, max=gate_clamp_upper_limit)
    if up_clamp_lower_limit is not None or up_clamp_upper_limit is not None:
        up = up.clamp(min=up_clamp_lower_limit, max=up_clamp_upper_limit)
    inter = up * _act(gate, hidden_act_fn)
    nxt = torch.einsum("eti,eih->eth", inter, expert_down_weights.to(torch.float32))
    if expert_down_bias is not None:
        nxt = nxt + expert_down_bias.unsqueeze(1).to(torch.float32)
    out = torch.zeros(T, H, dtype=torch.float32)
    if _name(expert_affinities_scaling_mode) == NO_SCALE:
        w = (aff > 0).to(torch.float32)
    else:
        w = aff
    for e in range(E_L):
        out = out + nxt[e] * w[:, e:e + 1]
    out = out.to(dtype)
    if skip_router_logits:
        return out
    return out, logits


def expert_mlp_fp32_routed(xn, aff, expert_gate_up_weights, expert_down_weights,
                           expert_gate_up_bias=None, expert_down_bias=None, hidden_act_fn=SILU,
                           gate_clamp_upper_limit=None, gate_clamp_lower_limit=None,
                           up_clamp_upper_limit=None, up_clamp_lower_limit=None,
                           scale_mode="POST_SCALE", out_dtype=None):
    """moe_block_tkg.py:223-297 on the selected experts only.  xn [T,H] (bf16),
    aff [T,E_L] fp32 (zeros for unselected).  Returns out in ``out_dtype`` (fp32 if
    None)."""
    T, H = xn.shape
    E_L, _, _, I = expert_gate_up_weights.shape
    x32 = xn.to(torch.float32)
    out = torch.zeros(T, H, dtype=torch.float32)
    w = (aff > 0).to(torch.float32) if _name(scale_mode) == NO_SCALE else aff
    for e in range(E_L):
        sel = torch.nonzero(aff[:, e] != 0).flatten()
        if sel.numel() == 0:
            continue
        gu = x32[sel] @ expert_gate_up_weights[e].reshape(H, 2 * I).to(torch.float32)
        if expert_gate_up_bias is not None:
            gu = gu + expert_gate_up_bias[e].reshape(2 * I).to(torch.float32)
        g, u = gu[:, :I], gu[:, I:]
        if gate_clamp_lower_limit is not None or gate_clamp_upper_limit is not None:
            g = g.clamp(min=gate_clamp_lower_limit, max=gate_clamp_upper_limit)
        if up_clamp_lower_limit is not None or up_clamp_upper_limit is not None:
            u = u.clamp(min=up_clamp_lower_limit, max=up_clamp_upper_limit)
        inter = u * _act(g, hidden_act_fn)
        y = inter @ expert_down_weights[e].to(torch.float32)
        if expert_down_bias is not None:
            y = y + expert_down_bias[e].to(torch.float32)
        term = torch.zeros(T, H, dtype=torch.float32)
        term[sel] = y * w[sel, e:e + 1]
        out = out + term
    return out if out_dtype is None else out.to(out_dtype)
