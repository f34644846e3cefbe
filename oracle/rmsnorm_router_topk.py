"""Oracle: fused RMSNorm + router top-k of the decode front end (quantization NONE).

Test infrastructure only (see ``oracle/__init__.py``).

Follows vllm_neuron/functional/moe/rmsnorm_router_topk_tkg.py ``_torch_impl``
(:214-279): RMSNorm in fp32 with the mean square taken over all H columns and divided
by hidden_actual (:249-254), the norm ``x * inv_rms * gamma`` cast to router_mm_dtype
(:256); the router operands cast to router_mm_dtype and multiplied with fp32
accumulation, the bias cast to router_mm_dtype and added in fp32 (:258-268); top-k on
the fp32 logits, the activation over the selected logits (:270-278), the result
scattered into bf16 affinities (:282-287).

Pinned by tests/test_oracle_norm.py: an fp64 closed form of the norm (per element,
rounded once to router_mm_dtype), of the logits (fp64 products of the cast operands) and
a brute-force top-k with math.exp / sigmoid over the selected values.
"""

from __future__ import annotations

import torch

SOFTMAX = "SOFTMAX"
SIGMOID = "SIGMOID"


def _name(v):
    return getattr(v, "name", v)


def rmsnorm_router_topk(hidden_states, gamma, router_weights, router_bias=None, eps=1e-6,
                        top_k=1, hidden_actual=None, router_mm_dtype=torch.bfloat16,
                        router_act_fn=SIGMOID):
    """rmsnorm_router_topk_tkg.py:214-279 with quantization_type NONE.  hidden_states
    [B, S, H]; gamma [1, H] or [H]; router_weights [H, E]; router_bias [1, E].
    Returns (norm [T, H] in router_mm_dtype, expert_index int32 [T, k], affinities bf16
    [T, E], logits fp32 [T, E])."""
    B, S, H = hidden_states.shape
    T = B * S
    x = hidden_states.to(torch.float32).reshape(T, H)
    g = gamma.to(torch.float32)
    if hidden_actual is not None:
        ss = torch.sum(x ** 2, dim=-1, keepdim=True)
        inv = torch.rsqrt(ss / hidden_actual + eps)
    else:
        inv = torch.rsqrt(torch.mean(x ** 2, dim=-1, keepdim=True) + eps)
    norm = (x * inv * g).to(router_mm_dtype)
    logits = norm.to(router_mm_dtype).float() @ router_weights.to(router_mm_dtype).float()
    if router_bias is not None:
        logits = logits + router_bias.to(router_mm_dtype).float()
    vals, idx = torch.topk(logits, k=top_k, dim=-1)
    fn = _name(router_act_fn)
    if fn == SOFTMAX:
        probs = torch.softmax(vals, dim=-1)
    elif fn == SIGMOID:
        probs = torch.sigmoid(vals)
    else:
        raise ValueError(f"Unsupported router_act_fn: {fn}")
    aff = torch.zeros(T, router_weights.shape[1], dtype=torch.bfloat16)
    aff.scatter_(-1, idx, probs.to(torch.bfloat16))
    return norm, idx.to(torch.int32), aff, logits
