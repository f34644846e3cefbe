"""Pins of oracle.blockwise: the torch flow vs a pure-Python closed form, plus invariants."""

import itertools

import pytest
import torch

from oracle import blockwise as ob


def random_affinities(T, E, K, g, zipf=None):
    logits = torch.randn(T, E, generator=g)
    if zipf:
        logits = logits - zipf * torch.log1p(torch.arange(E, dtype=torch.float32))
    vals, idx = torch.topk(logits, K, dim=1)
    aff = torch.zeros(T, E)
    aff.scatter_(1, idx, torch.softmax(vals, 1))
    return aff


def check_invariants(aff, tp2id, b2e, cond, E, B):
    T = aff.shape[0]
    N = b2e.numel()
    assert tp2id.numel() == N * B
    slots = tp2id.view(N, B)
    seen = set()
    for n in range(N):
        for s in slots[n].tolist():
            if s >= 0:
                e = int(b2e[n])
                assert aff[s, e] != 0
                assert (s, e) not in seen
                seen.add((s, e))
    assert seen == {(t, e) for t in range(T) for e in range(E) if aff[t, e] != 0}
    assert torch.all(b2e[1:] >= b2e[:-1])
    assert torch.equal(cond, (slots != -1).any(1).to(torch.int32))
    # ascending tokens inside each expert's run
    for e in range(E):
        run = [s for n in range(N) if b2e[n] == e for s in slots[n].tolist() if s >= 0]
        assert run == sorted(run)


@pytest.mark.parametrize("T,E,K,B", [(1, 4, 2, 4), (3, 3, 1, 2), (5, 4, 4, 2), (9, 2, 1, 4)])
def test_exhaustive_tiny_masks(T, E, K, B):
    # every row is any K-subset of experts: enumerate all combinations for small T*E
    subsets = list(itertools.combinations(range(E), K))
    g = torch.Generator().manual_seed(T * 100 + E)
    picks = torch.randint(0, len(subsets), (200, T), generator=g)
    for trial in range(picks.shape[0]):
        aff = torch.zeros(T, E)
        for t in range(T):
            for e in subsets[int(picks[trial, t])]:
                aff[t, e] = 0.5
        _, tp2id, b2e, cond = ob.build_blockwise_mapping(aff, E, K, B)
        lt, lb, lc = ob.build_blockwise_mapping_loops(aff, E, K, B)
        assert torch.equal(tp2id, lt) and torch.equal(b2e, lb) and torch.equal(cond, lc)


@pytest.mark.parametrize("T,E,K,B,zipf", [(64, 8, 2, 16, None), (200, 32, 4, 32, 1.2),
                                          (257, 16, 1, 128, None), (100, 5, 5, 8, None)])
def test_random_vs_loops_and_invariants(T, E, K, B, zipf):
    g = torch.Generator().manual_seed(T + E)
    aff = random_affinities(T, E, K, g, zipf)
    am, tp2id, b2e, cond = ob.build_blockwise_mapping(aff, E, K, B)
    lt, lb, lc = ob.build_blockwise_mapping_loops(aff, E, K, B)
    assert torch.equal(tp2id, lt) and torch.equal(b2e, lb) and torch.equal(cond, lc)
    assert torch.equal(am.view(T, E), aff)
    check_invariants(aff, tp2id, b2e, cond, E, B)


def test_num_blocks_bound():
    assert ob.num_blocks(4096, 32, 4, 256) == 95
    assert ob.num_blocks(4096, 128, 4, 256) == 191
    assert ob.num_blocks(8192, 256, 8, 256) == 511
    assert ob.num_blocks(1, 32, 4, 256) == 4
    # the bound holds for the worst case: E-1 experts with one token each
    T, E, K, B = 40, 8, 2, 16
    aff = torch.zeros(T, E)
    aff[:, 0] = 1.0
    for t in range(E - 1):
        aff[t, t + 1] = 1.0
    aff[E - 1:, 1] = 1.0
    _, tp2id, b2e, cond = ob.build_blockwise_mapping(aff, E, K, B)
    check_invariants(aff, tp2id, b2e, cond, E, B)


def test_padding_mask_only_scales_affinities():
    g = torch.Generator().manual_seed(9)
    aff = random_affinities(20, 4, 2, g)
    pm = torch.arange(20) < 13
    am, tp2id, b2e, cond = ob.build_blockwise_mapping(aff, 4, 2, 8, padding_mask=pm)
    _, tp2, b2, c2 = ob.build_blockwise_mapping(aff, 4, 2, 8)
    assert torch.equal(tp2id, tp2) and torch.equal(b2e, b2)
    assert torch.equal(am.view(20, 4), aff * pm.float().unsqueeze(1))


def test_cumsum_matmul_chunks():
    g = torch.Generator().manual_seed(2)
    t = (torch.rand(5000, 3, generator=g) < 0.3).float()
    assert torch.equal(ob.cumsum_matmul(t), torch.cumsum(t, 0))
