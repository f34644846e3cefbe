"""Pins of oracle.router against an fp64 brute force and the routing invariants."""

import math

import pytest
import torch

from oracle import router as orr


def brute(x, w_he, k, bias, act):
    T, E = x.shape[0], w_he.shape[1]
    xd, wd = x.double(), w_he.double()
    aff = torch.zeros(T, E, dtype=torch.float64)
    for t in range(T):
        logits = [sum(float(xd[t, h]) * float(wd[h, e]) for h in range(x.shape[1]))
                  + (float(bias[e]) if bias is not None else 0.0) for e in range(E)]
        order = sorted(range(E), key=lambda e: (-logits[e], e))[:k]
        vals = [logits[e] for e in order]
        if act == "softmax":
            m = max(vals)
            ex = [math.exp(v - m) for v in vals]
            probs = [v / sum(ex) for v in ex]
        else:
            probs = [1.0 / (1.0 + math.exp(-v)) for v in vals]
        for e, p in zip(order, probs):
            aff[t, e] = p
    return aff


@pytest.mark.parametrize("act", ["softmax", "sigmoid"])
@pytest.mark.parametrize("E,k", [(8, 2), (16, 4), (6, 6)])
def test_router_matches_fp64_brute_force(act, E, k):
    g = torch.Generator().manual_seed(E * 10 + k)
    T, H = 7, 40
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = (torch.randn(E, H, generator=g) * 0.3).to(torch.bfloat16)
    b = (torch.randn(E, generator=g) * 0.1).to(torch.bfloat16)
    aff = orr.router(x, w.T, k, b, act)
    want = brute(x, w.T, k, b, act)
    assert torch.equal(aff != 0, want != 0)
    assert torch.allclose(aff.double(), want, rtol=1e-5, atol=1e-7)


def test_router_invariants():
    g = torch.Generator().manual_seed(3)
    T, H, E, k = 64, 128, 32, 4
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)
    aff, logits = orr.router(x, w.T, k, return_logits=True)
    assert aff.dtype == torch.float32 and logits.shape == (T, E)
    assert torch.all((aff != 0).sum(1) == k)
    assert torch.allclose(aff.sum(1), torch.ones(T), atol=1e-6)
    sel = aff != 0
    min_sel = torch.where(sel, logits, torch.full_like(logits, float("inf"))).min(1).values
    max_uns = torch.where(~sel, logits, torch.full_like(logits, -float("inf"))).max(1).values
    assert torch.all(min_sel >= max_uns)


def test_renorm_and_scatter_act_orders():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(5, 32, generator=g).to(torch.bfloat16)
    w = torch.randn(8, 32, generator=g).to(torch.bfloat16)
    a0 = orr.router(x, w.T, 3, router_computation_order=orr.PRENORM_LINEAR_TOPK_ACT_SCATTER)
    a1 = orr.router(x, w.T, 3, router_computation_order=orr.PRENORM_LINEAR_ACT_TOPK_RENORM_SCATTER)
    a2 = orr.router(x, w.T, 3, router_computation_order=orr.PRENORM_LINEAR_TOPK_SCATTER_ACT)
    # softmax over all then top-k + L1 renorm equals softmax over the top-k
    assert torch.allclose(a0, a1, atol=1e-6)
    # scatter into -inf then softmax over the row equals softmax over the top-k
    assert torch.allclose(a0, a2, atol=1e-6)


def test_validation_errors():
    x = torch.zeros(2, 8, dtype=torch.bfloat16)
    w = torch.zeros(8, 4, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        orr.router(x, w, 5)
    with pytest.raises(ValueError):
        orr.router(x, torch.zeros(7, 4, dtype=torch.bfloat16), 2)
