"""Blockwise mapping kernel vs the oracle's torch flow: bit-exact on every output."""

import pytest
import torch

from oracle import blockwise as ob

pytestmark = pytest.mark.gpu


def _aff(T, E, K, seed, zipf=None, exact_zero_rows=0):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, E, generator=g)
    if zipf:
        perm = torch.randperm(E, generator=g)
        logits = logits - zipf * torch.log1p(perm.float())
    vals, idx = torch.topk(logits, K, dim=1)
    aff = torch.zeros(T, E)
    aff.scatter_(1, idx, torch.softmax(vals, 1))
    if exact_zero_rows:
        aff[:exact_zero_rows] = 0.0
    return aff


CASES = [
    (1, 32, 4, 256, None), (4, 32, 4, 256, None), (64, 128, 4, 256, None),
    (4096, 32, 4, 256, None), (4096, 32, 4, 256, 1.2), (4096, 128, 4, 256, None),
    (8192, 256, 8, 256, 1.0), (300, 7, 3, 128, None), (257, 1, 1, 128, None),
    (1000, 16, 16, 128, None), (16384, 64, 2, 512, 2.0),
    # the largest expert count the kernels take (1,024), and a large one that is not a
    # multiple of 4 (affinity rows read one element at a time)
    (96, 1024, 8, 128, None), (130, 1001, 8, 256, 1.0),
    # over 32K chunk masks (65 chunks x 512 experts): the scan and scatter kernels instead
    # of the one placement kernel
    (4160, 512, 4, 256, None),
]


@pytest.mark.parametrize("T,E,K,B,zipf", CASES)
def test_blockwise_bit_exact(dev, T, E, K, B, zipf):
    from vllm_neuron_amd import functional as NF

    aff = _aff(T, E, K, T * 7 + E, zipf, exact_zero_rows=3 if T > 10 else 0)
    am_r, tp_r, b2e_r, c_r = ob.build_blockwise_mapping(aff, E, K, B)
    am_g, tp_g, b2e_g, c_g = NF.build_blockwise_mapping(aff.to(dev), E, K, B)
    assert torch.equal(am_g.cpu(), am_r)
    assert torch.equal(tp_g.cpu(), tp_r)
    assert torch.equal(b2e_g.cpu(), b2e_r)
    assert torch.equal(c_g.cpu(), c_r)


@pytest.mark.parametrize("T,E", [(777, 32), (4160, 512)])
def test_blockwise_padding_mask(dev, T, E):
    from vllm_neuron_amd import functional as NF

    K, B = 4, 256
    aff = _aff(T, E, K, 5)
    pm = torch.arange(T) <= 2 * T // 3
    r = ob.build_blockwise_mapping(aff, E, K, B, padding_mask=pm)
    g = NF.build_blockwise_mapping(aff.to(dev), E, K, B, padding_mask=pm.to(dev))
    for a, b in zip(g, r):
        assert torch.equal(a.cpu(), b)
