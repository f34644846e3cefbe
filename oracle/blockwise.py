"""Oracle: blockwise token -> expert mapping (the permutation), torch flow.

Test infrastructure only (see ``oracle/__init__.py``).

Follows vllm_neuron/functional/moe/moe_blockwise.py:
  * ``build_blockwise_mapping``  <- ``build_blockwise_mapping`` (:24-156) on its torch
                                    branch ``_build_blockwise_mapping_torch`` (:294-400)
                                    at tp_degree = 1 (one rank, no collectives)
  * ``cumsum_matmul``            <- ``_cumsum_matmul`` (:403-440)
  * ``apply_padding_mask``       <- ``_apply_padding_mask`` (:443-461)

Pinned by (tests/test_oracle_blockwise.py): ``build_blockwise_mapping_loops``,
a pure-Python restatement from the closed form (stable counting sort by expert
with every expert's run padded to a multiple of the block size; ``N`` from the
bound at :343-349; trailing empty blocks owned by expert E-1), compared on
exhaustive tiny cases and random small ones, plus the invariants: every routed
(t, e) appears exactly once, ascending t inside an expert, -1 padding,
non-decreasing ``block_to_expert``, ``conditions`` = block holds a token.
"""

from __future__ import annotations

import math
from typing import Optional

import torch


def cumsum_matmul(t: torch.Tensor, tril_size: int = 2048) -> torch.Tensor:
    """moe_blockwise.py:403-440: inclusive cumsum over dim 0 as fp32 lower-triangular
    matmuls in chunks of ``tril_size`` rows with a rolling carry; exact for counts
    below 2^24."""
    n = t.shape[0]
    if n % tril_size == 0:
        iters, last = n // tril_size, tril_size
    else:
        iters, last = n // tril_size + 1, n % tril_size
    outs = []
    carry = torch.zeros(1, t.shape[1], dtype=torch.float32)
    for i in range(iters):
        m = tril_size if i < iters - 1 else last
        tril = torch.tril(torch.ones(m, m, dtype=torch.float32))
        o = carry + tril @ t.narrow(0, i * tril_size, m).to(torch.float32)
        outs.append(o)
        if i < iters - 1:
            carry = o.narrow(0, -1, 1)
    return torch.cat(outs, dim=0).to(t.dtype)


def apply_padding_mask(aff: torch.Tensor, padding_mask: Optional[torch.Tensor]) -> torch.Tensor:
    """moe_blockwise.py:443-461."""
    if padding_mask is None:
        return aff
    return aff * padding_mask.float().unsqueeze(1)


def num_blocks(T: int, E: int, K: int, B: int) -> int:
    """moe_blockwise.py:343-349: the worst-case block count for T*min(K,E) routed pairs."""
    total = T * min(K, E)
    n = math.ceil((total - (E - 1)) / B) + E - 1
    return min(n, total)


def build_blockwise_mapping(expert_affinities: torch.Tensor, num_local_experts: int,
                            num_experts_per_token: int, block_size: int,
                            padding_mask: Optional[torch.Tensor] = None):
    """moe_blockwise.py:24-156 + :294-400 (tp_degree = 1).

    Returns (affinities_masked [T*E, 1], token_position_to_id [N*B] int32,
    block_to_expert [N] int32, conditions [N] int32).
    """
    T = expert_affinities.shape[0]
    E = num_local_experts
    B = block_size
    mask = (expert_affinities != 0).to(torch.float32)
    aff_masked = apply_padding_mask(expert_affinities, padding_mask).view(-1, 1)

    tokens_per_expert = torch.sum(mask, dim=0)
    blocks_per_expert = ((tokens_per_expert + B - 1) // B).to(torch.long)
    N = num_blocks(T, E, num_experts_per_token, B)
    block_ids = torch.arange(N, dtype=torch.long)
    cum_blocks = cumsum_matmul(blocks_per_expert.unsqueeze(1)).squeeze(1)
    block_to_expert = torch.sum(block_ids.unsqueeze(1) >= cum_blocks[:-1], dim=1).to(torch.long)

    pos = cumsum_matmul(mask)  # [T, E], 1-based rank of t among e's tokens
    offsets = cum_blocks * B
    pos[:, 1:] += offsets[:-1]
    pos = pos.masked_fill(mask == 0, 0).to(torch.long)
    tok = torch.arange(T, dtype=torch.long)
    tp2id = -1 * torch.ones(N * B + 1, dtype=torch.long)
    tp2id[pos] = tok.unsqueeze(1).expand(T, E)
    tp2id = tp2id[1:]

    conditions = torch.any(tp2id.view(N, B) != -1, dim=1).to(torch.int32)
    return aff_masked, tp2id.to(torch.int32), block_to_expert.to(torch.int32), conditions


def build_blockwise_mapping_loops(expert_affinities: torch.Tensor, num_local_experts: int,
                                  num_experts_per_token: int, block_size: int):
    """Closed-form restatement with plain Python loops (small inputs only): a stable
    counting sort of routed (t, e) pairs by expert, each expert's run padded with -1
    to a multiple of ``block_size``, runs laid out in expert order, then -1 blocks up
    to the bound ``N``; block n belongs to the expert whose run covers it, and blocks
    past the last run belong to expert E-1."""
    T = expert_affinities.shape[0]
    E = num_local_experts
    B = block_size
    a = expert_affinities.tolist()
    N = num_blocks(T, E, num_experts_per_token, B)
    slots = []
    owner = []
    for e in range(E):
        toks = [t for t in range(T) if a[t][e] != 0]
        nb = (len(toks) + B - 1) // B
        run = toks + [-1] * (nb * B - len(toks))
        slots += run
        owner += [e] * nb
    assert len(owner) <= N
    slots += [-1] * (N * B - len(slots))
    owner += [E - 1] * (N - len(owner))
    cond = [int(any(s != -1 for s in slots[n * B:(n + 1) * B])) for n in range(N)]
    return (torch.tensor(slots, dtype=torch.int32), torch.tensor(owner, dtype=torch.int32),
            torch.tensor(cond, dtype=torch.int32))
