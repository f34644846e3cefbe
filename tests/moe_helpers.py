"""Shared helpers of the MoE parity tests (GPU layer vs oracle layer)."""

from __future__ import annotations

import torch

# Layer-output tolerance: max|d| / max|ref| and mean|d| / mean|ref| (the normalization
# of the reference's accuracy/testing.py:117-205 assert_close).
MAX_REL = 2e-2
MEAN_REL = 5e-3


def build(shape, seed, dev, E=None, exp=(120, 130), zipf=None):
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.layer import MXFP4MoE
    from vllm_neuron_amd.weights import MXFP4Experts

    from oracle.layer import RefLayer

    lt = synthetic.layer_tensors(shape, seed, zipf_s=zipf, exp_range=exp, E=E)
    ref = RefLayer(lt)
    w = MXFP4Experts.from_checkpoint(lt.gate_up_blocks, lt.gate_up_scales, lt.down_blocks,
                                     lt.down_scales, lt.gate_up_bias, lt.down_bias).to(dev)
    rb = None if lt.router_b is None else lt.router_b.to(dev)
    layer = MXFP4MoE(w, lt.router_w.to(dev), rb, shape.K, shape.swiglu_limit)
    return ref, layer, lt


def routing_agreement(layer, ref, x, dev):
    """GPU routing vs oracle routing; returns (oracle affinities, mask of tokens whose
    selected set differs only through a near-tie)."""
    aff_g, logits_g, _, _ = layer.route(x.to(dev))
    aff_r, logits_r = ref.route(x)
    aff_g, logits_g = aff_g.cpu(), logits_g.cpu()
    assert torch.allclose(logits_g, logits_r, rtol=1e-5, atol=1e-5)
    bad = ((aff_g != 0) != (aff_r != 0)).any(1)
    k = ref.K
    for t in torch.nonzero(bad).flatten().tolist():
        srt = torch.sort(logits_r[t], descending=True).values
        assert (srt[k - 1] - srt[k]).abs() < 1e-5 * max(1.0, srt[0].abs().item())
    return aff_r, bad


def routing_from_logits(logits_g, ref, x):
    """Like routing_agreement, for logits a fused GPU call returned (logits_out)."""
    aff_r, logits_r = ref.route(x)
    logits_g = logits_g.cpu()
    assert torch.allclose(logits_g, logits_r, rtol=1e-5, atol=1e-5)
    k = ref.K
    sel_g = torch.zeros_like(logits_g, dtype=torch.bool)
    sel_g.scatter_(1, torch.topk(logits_g, k, dim=1).indices, True)
    bad = (sel_g != (aff_r != 0)).any(1)
    for t in torch.nonzero(bad).flatten().tolist():
        srt = torch.sort(logits_r[t], descending=True).values
        assert (srt[k - 1] - srt[k]).abs() < 1e-5 * max(1.0, srt[0].abs().item())
    return aff_r, bad


def check_close(got, want, skip_rows=None, label=""):
    got = got.double()
    want = want.double()
    if skip_rows is not None and skip_rows.any():
        keep = ~skip_rows
        got, want = got[keep], want[keep]
    d = (got - want).abs()
    mx = (d.max() / want.abs().max()).item()
    mean = (d.mean() / want.abs().mean()).item()
    exact = (d == 0).double().mean().item()
    print(f"{label}: max|d|/max|ref|={mx:.3e} mean|d|/mean|ref|={mean:.3e} "
          f"raw max|d|={d.max().item():.4g} max|ref|={want.abs().max().item():.4g} "
          f"bit-identical={exact:.4f}")
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)
    return mx, mean
