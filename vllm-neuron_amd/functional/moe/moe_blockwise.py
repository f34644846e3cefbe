"""Blockwise token -> expert mapping on the MI355X kernel.

Mirrors vllm_neuron/functional/moe/moe_blockwise.py:24-156 (signature and return
values).  The reference runs nkilib find_nonzero_indices + indexed_flatten
(:159-291) or its torch flow (:294-400); here mxmoe_blockwise_mapping produces the
same four tensors bit for bit.  Tensor-parallel sharding of the mapping
(tp_degree > 1, moe_group collectives) is multi-GPU and raises NotImplementedError.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
from torch import Tensor

from ... import _lib


def num_blocks(T: int, E: int, K: int, block_size: int) -> int:
    """Worst-case block count (moe_blockwise.py:343-349)."""
    total = T * min(K, E)
    n = math.ceil((total - (E - 1)) / block_size) + E - 1
    return min(n, total)


def build_blockwise_mapping(expert_affinities: Tensor, num_local_experts: int,
                            num_experts_per_token: int, block_size: int, moe_group=None,
                            tp_degree: int = 1, padding_mask: Optional[Tensor] = None,
                            return_expert_counts: bool = False):
    """expert_affinities fp32 [T, E_local] (zeros for unselected experts) ->
    (expert_affinities_masked [T*E, 1] fp32, token_position_to_id [N*B] int32,
    block_to_expert [N] int32, conditions [N] int32)."""
    if tp_degree > 1:
        raise NotImplementedError("tensor-parallel blockwise mapping needs several GPUs")
    if expert_affinities.dim() != 2 or expert_affinities.shape[1] != num_local_experts:
        raise ValueError(f"expected expert_affinities [T, {num_local_experts}], got "
                         f"{tuple(expert_affinities.shape)}")
    dev = _lib.require_cuda(expert_affinities, padding_mask)
    aff = expert_affinities
    if aff.dtype != torch.float32:
        aff = aff.to(torch.float32)
    aff = aff.contiguous()
    T, E = aff.shape
    N = num_blocks(T, E, num_experts_per_token, block_size)
    pm = None
    if padding_mask is not None:
        pm = padding_mask.to(torch.uint8).contiguous()
    aff_masked = torch.empty(T * E, 1, dtype=torch.float32, device=dev)
    tp2id = torch.empty(N * block_size, dtype=torch.int32, device=dev)
    b2e = torch.empty(N, dtype=torch.int32, device=dev)
    cond = torch.empty(N, dtype=torch.int32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    L = _lib.lib()
    ws = _lib.workspace(L.mxmoe_blockwise_workspace_bytes(T, E), dev)
    rc = L.mxmoe_blockwise_mapping(aff.data_ptr(), _lib.ptr(pm), T, E, num_experts_per_token,
                                   block_size, N, aff_masked.data_ptr(), tp2id.data_ptr(),
                                   b2e.data_ptr(), cond.data_ptr(), counts.data_ptr(),
                                   ws.data_ptr(), ws.numel(), _lib.stream_handle(dev))
    _lib.check(rc, "mxmoe_blockwise_mapping")
    out = (aff_masked, tp2id, b2e, cond)
    return out + (counts,) if return_expert_counts else out
