"""Shared helpers of the MoE parity tests (GPU layer vs oracle layer)."""

from __future__ import annotations

import torch

# Layer-output tolerance: max|d| / max|ref| and mean|d| / mean|ref| (the normalization
# of the reference's accuracy/testing.py:117-205 assert_close).
MAX_REL = 2e-2
MEAN_REL = 5e-3


def build(shape, seed, dev, E=None, exp=(120, 130), zipf=None, lazy=False, pack_on_gpu=False):
    """(oracle layer, GPU layer, checkpoint tensors) of one synthetic layer; lazy: the
    oracle dequantizes each expert when a routed form first needs it; pack_on_gpu: the
    checkpoint tensors are packed into the kernel layout on the GPU (large layers)."""
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.layer import MXFP4MoE
    from vllm_neuron_amd.weights import MXFP4Experts

    from oracle.layer import RefLayer

    lt = synthetic.layer_tensors(shape, seed, zipf_s=zipf, exp_range=exp, E=E)
    ref = RefLayer(lt, lazy=lazy)
    if pack_on_gpu:
        mv = lambda t: None if t is None else t.to(dev)  # noqa: E731
        w = MXFP4Experts.from_checkpoint(mv(lt.gate_up_blocks), mv(lt.gate_up_scales),
                                         mv(lt.down_blocks), mv(lt.down_scales),
                                         mv(lt.gate_up_bias), mv(lt.down_bias))
    else:
        w = MXFP4Experts.from_checkpoint(lt.gate_up_blocks, lt.gate_up_scales, lt.down_blocks,
                                         lt.down_scales, lt.gate_up_bias, lt.down_bias).to(dev)
    rb = None if lt.router_b is None else lt.router_b.to(dev)
    layer = MXFP4MoE(w, lt.router_w.to(dev), rb, shape.K, shape.swiglu_limit)
    return ref, layer, lt


def routing_agreement(layer, ref, x, dev):
    """GPU router (logits, selected experts in order, affinities) vs the oracle's routing;
    returns (oracle affinities, mask of tokens that differ only through a near-tie)."""
    aff_g, logits_g, idx_g, _ = layer.route(x.to(dev))
    aff_r, logits_r = ref.route(x)
    aff_g, logits_g = aff_g.cpu(), logits_g.cpu()
    assert torch.allclose(logits_g, logits_r, rtol=1e-5, atol=1e-5)
    k = ref.K
    idx_r = torch.topk(logits_r, k, dim=1).indices
    bad = check_indices(idx_g, logits_r, idx_r, k, "router")
    bad |= ((aff_g != 0) != (aff_r != 0)).any(1)
    for t in torch.nonzero(bad).flatten().tolist():
        assert near_tie(logits_r[t], k)
    ok = ~bad
    aff_close(aff_g[ok], aff_r[ok], logits_g[ok], logits_r[ok], 1e-6)
    return aff_r, bad


def aff_close(aff_g, aff_r, logits_g, logits_r, tol):
    """Affinities within tol (one rounding step of the computation dtype below 1) plus the
    token's largest logit difference (a softmax or sigmoid moves by less than its input)."""
    dl = (logits_g.double() - logits_r.double()).abs().max(1, keepdim=True).values
    d = (aff_g.double() - aff_r.double()).abs()
    assert bool((d <= tol + dl).all()), float((d - tol - dl).max())


def near_tie(scores, k, rel=1e-5):
    """Sorted scores of one token: whether two of the first k + 1 lie within the fp32
    summation-order error, so that two correct implementations may pick or order them
    differently."""
    srt = torch.sort(scores, descending=True).values.double()
    scale = max(1.0, srt[0].abs().item())
    gaps = (srt[:k] - srt[1:k + 1]).abs()
    return bool((gaps < rel * scale).any())


def check_indices(idx_g, scores_r, idx_r, k, label="", rel=1e-5):
    """The experts a GPU front end selected (idx_g [T, k], descending) equal the oracle's
    (idx_r) element for element; a token may differ only through a near-tie of the
    oracle's scores within rel (counted, printed, and returned as a mask).  rel covers
    the fp32 summation-order error of the logits (1e-5), or, behind an RMSNorm, one bf16
    rounding step of a normalized element times a router weight (2e-4)."""
    idx_g, idx_r = idx_g.cpu().long(), idx_r.cpu().long()
    bad = (idx_g != idx_r).any(1)
    for t in torch.nonzero(bad).flatten().tolist():
        assert near_tie(scores_r[t], k, rel), f"{label} token {t}: {idx_g[t].tolist()} vs " \
                                               f"{idx_r[t].tolist()}"
    print(f"{label}: top-k indices identical on {int((~bad).sum())} of {len(bad)} tokens, "
          f"near-ties {int(bad.sum())}")
    return bad


def routing_from_logits(logits_g, ref, x, idx_g=None):
    """GPU front-end outputs (logits_out, and topk_idx_out when given) against the
    oracle's routing: logits within fp32 summation error, the selected experts exactly
    (near-ties exempted and counted).  Returns (oracle affinities, exempted tokens)."""
    aff_r, logits_r = ref.route(x)
    logits_g = logits_g.cpu()
    assert torch.allclose(logits_g, logits_r, rtol=1e-5, atol=1e-5)
    k = ref.K
    idx_r = torch.topk(logits_r, k, dim=1).indices
    if idx_g is None:  # only the logits came back: check the selection they imply
        idx_g = torch.topk(logits_g, k, dim=1).indices
    bad = check_indices(idx_g, logits_r, idx_r, k, "front end")
    return aff_r, bad


def decode_checked(layer, ref, x, dev):
    """One mxmoe_moe_decode call with the front end's logits and selected experts returned,
    both checked against the oracle.  Returns (output [T, H] on the CPU, oracle affinities,
    near-tie tokens)."""
    T = x.shape[0]
    logits = torch.empty(T, ref.E, dtype=torch.float32, device=dev)
    idx = torch.empty(T, ref.K, dtype=torch.int32, device=dev)
    got = layer.decode(x.to(dev), logits_out=logits, topk_idx_out=idx).cpu()
    aff, ties = routing_from_logits(logits, ref, x, idx)
    return got, aff, ties


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
