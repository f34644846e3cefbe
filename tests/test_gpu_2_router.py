"""Router kernel vs the oracle's torch flow.

Indices must match exactly; the only tolerated difference is a near-tie between the
k-th and (k+1)-th logit smaller than the fp32 summation-order error of the two
implementations (both sum exact bf16 products in fp32, in different orders), which is
counted and reported.  Affinities agree to fp32 rounding."""

import pytest
import torch

from oracle import router as orr
from oracle import moe_block_tkg as obt

pytestmark = pytest.mark.gpu


def _inputs(T, E, H, seed, zipf=None):
    from vllm_neuron_amd import synthetic

    x = synthetic.normal_bf16(seed, (T, H))
    w = synthetic.normal_bf16(seed + 1, (E, H), 0.02)
    b = synthetic.zipf_bias(seed + 2, E, zipf) if zipf else None
    return x, w, b


def compare_routing(aff_g, logits_g, aff_r, logits_r, k):
    assert torch.allclose(logits_g, logits_r, rtol=1e-5, atol=1e-5), \
        (logits_g - logits_r).abs().max()
    sel_g, sel_r = aff_g != 0, aff_r != 0
    bad = (sel_g != sel_r).any(1)
    ties = 0
    for t in torch.nonzero(bad).flatten().tolist():
        srt = torch.sort(logits_r[t], descending=True).values
        gap = (srt[k - 1] - srt[k]).abs().item()
        assert gap < 1e-5 * max(1.0, srt[0].abs().item()), f"token {t}: gap {gap}"
        ties += 1
    ok = ~bad
    assert torch.allclose(aff_g[ok], aff_r[ok], rtol=2e-6, atol=1e-7)
    return ties


@pytest.mark.parametrize("T,E,k,H", [(1, 32, 4, 2880), (64, 128, 4, 2880), (4096, 32, 4, 2880),
                                     (4096, 128, 4, 2880), (128, 256, 8, 7168), (17, 8, 2, 64),
                                     (64, 512, 4, 256), (33, 300, 8, 128), (1000, 1024, 8, 256),
                                     (1030, 100, 4, 256)])
def test_router_softmax(dev, T, E, k, H):
    from vllm_neuron_amd import functional as NF

    x, w, _ = _inputs(T, E, H, 100 + E + T)
    aff_g, logits_g = NF.router(x.to(dev), w.to(dev).T, k, return_logits=True)
    aff_r, logits_r = orr.router(x, w.T, k, return_logits=True)
    ties = compare_routing(aff_g.cpu(), logits_g.cpu(), aff_r, logits_r, k)
    print(f"T={T} E={E} k={k}: near-ties {ties}")
    assert ties <= max(1, T // 1000)


@pytest.mark.parametrize("order", ["PRENORM_LINEAR_ACT_TOPK_RENORM_SCATTER",
                                   "PRENORM_LINEAR_TOPK_SCATTER_ACT"])
@pytest.mark.parametrize("act", ["softmax", "sigmoid"])
def test_router_orders_and_bias(dev, order, act):
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd.enums import RouterComputationOrder

    T, E, k, H = 300, 32, 4, 2880
    x, w, b = _inputs(T, E, H, 7, zipf=1.2)
    o = RouterComputationOrder[order]
    aff_g, logits_g = NF.router(x.to(dev), w.to(dev).T, k, router_bias=b.to(dev), activation=act,
                                return_logits=True, router_computation_order=o)
    aff_r, logits_r = orr.router(x, w.T, k, b, act, return_logits=True,
                                 router_computation_order=o.value)
    compare_routing(aff_g.cpu(), logits_g.cpu(), aff_r, logits_r, k)


def test_rmsnorm_router_block_tkg_front_end(dev):
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd.functional.moe.router import router_topk_raw

    T, E, k, H = 64, 128, 4, 2880
    x, w, _ = _inputs(T, E, H, 9)
    gamma = (1.0 + 0.1 * torch.randn(H, generator=torch.Generator().manual_seed(1))).float()
    xn_g = NF.rmsnorm(x.to(dev), gamma.to(dev), 1e-5, hidden_actual=2800).cpu()
    xn_r, logits_r, top_r, idx_r = obt.rmsnorm_router(x, gamma, w.T, None, 1e-5, k, "SOFTMAX",
                                                      False, True, hidden_actual=2800)
    d = (xn_g.float() - xn_r.float()).abs()
    # one bf16 ulp of each reference value (the fp32 variance sums in another order)
    ulp = torch.ldexp(torch.ones_like(d), torch.frexp(xn_r.float()).exponent - 8)
    assert torch.all(d <= ulp), d.max()
    assert (d == 0).float().mean() > 0.99
    # router stage on the reference's normalized rows, with renorm (+1e-20)
    _, logits_g, idx_g, val_g = router_topk_raw(xn_r.to(dev), w.to(dev), k, None, 0, False, True,
                                                1e-20)
    assert torch.allclose(logits_g.cpu(), logits_r, rtol=1e-5, atol=1e-5)
    assert torch.equal(idx_g.cpu().long(), idx_r)
    assert torch.allclose(val_g.cpu(), top_r, rtol=2e-6, atol=1e-7)
