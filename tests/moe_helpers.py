"""Shared helpers of the MoE parity tests (GPU layer vs oracle layer)."""

from __future__ import annotations

import torch

# Layer-output tolerance: max|d| / max|ref| and mean|d| / mean|ref| (the normalization
# of the reference's accuracy/testing.py:117-205 assert_close).
MAX_REL = 2e-2
MEAN_REL = 5e-3
# Regression bounds at the level the kernels reach (far inside the tolerance above):
# bf16 outputs (decode: bf16 of an fp32 computation, as the reference's decode flow;
# prefill: bf16 of the fp32 combine) agree with
# the oracle bit for bit on at least 99.5 % of the elements (measured 99.6-99.9 %), and
# no element differs by more than one bf16 step of its row's largest output (the final
# rounding of a sum whose fp32 value differs in the last bits; an element that nearly
# cancels can be many of its own steps away, which is why the step of the row is used);
# prefill outputs in fp32 differ from the oracle's only through the order of fp32 sums
# inside the GEMMs (a different rounding of a bf16 intermediate now and then): measured
# mean|d|/mean|ref| 5.8-7.2e-6 on the GPT-OSS shapes (clamped SwiGLU), 1.4e-5 on the
# 256-expert shape (plain SwiGLU, outputs up to 6e8).  Planted in a CPU copy of the flow
# (GPT-OSS-20B shape, 8 experts, 256 tokens): gate/up GEMM outputs kept in fp32 instead
# of bf16 give mean 3.6e-4 and 89.7 % bit-identical bf16 outputs, far outside both
# bounds; the down output rounded once instead of before and after its bias (which is
# small next to it) stays inside them (6.6e-6, 99.8 %), as the flows rarely differ.
BF16_OUT = (0.995, 1)
PREFILL_FP32_MEAN = 1e-5
PREFILL_FP32_MEAN_PLAIN = 3e-5


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


def bf16_ulp_distance(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Elementwise distance in bf16 units in the last place between two bf16 tensors (the
    difference of their bit patterns on the number line; +0 and -0 coincide)."""
    def ordered(t):
        v = t.contiguous().view(torch.int16).to(torch.int32)
        return torch.where(v < 0, -(v & 0x7FFF), v)
    return (ordered(a) - ordered(b)).abs()


def bf16_step(v: torch.Tensor) -> torch.Tensor:
    """The spacing of bf16 numbers at |v| (normal range): 2^(floor(log2 |v|) - 7)."""
    _, e = torch.frexp(v.double().abs().clamp_min(2.0 ** -126))
    return torch.ldexp(torch.ones_like(v, dtype=torch.float64), e - 8)


def stratified_rows(aff: torch.Tensor, extra: int = 0, seed: int = 0, tile: int = 128):
    """Token rows that reach every M-tile of the prefill GEMMs: for each expert, its first
    and last token and the tokens on both sides of every 128-slot tile boundary (tokens
    sit in ascending order within an expert's blocks), so that full tiles, nearly empty
    second tiles and a hot expert's multi-block runs are all checked; plus ``extra``
    random rows."""
    mask = aff != 0
    T = aff.shape[0]
    pick = set()
    for e in range(aff.shape[1]):
        toks = torch.nonzero(mask[:, e]).flatten()
        c = len(toks)
        if c == 0:
            continue
        js = {0, c - 1}
        for m in range(1, (c + tile - 1) // tile):
            js.update((tile * m - 1, tile * m))
        pick.update(int(toks[j]) for j in js if j < c)
    if extra:
        g = torch.Generator().manual_seed(seed)
        pick.update(torch.randint(0, T, (extra,), generator=g).tolist())
    return torch.tensor(sorted(pick), dtype=torch.long)


def check_close(got, want, skip_rows=None, label="", mean_bound=None, ulp=None):
    """Layer outputs against the oracle.  Always: the normalized bounds (max 2e-2, mean
    5e-3).  mean_bound: a tighter bound on the normalized mean error at the level the
    kernels achieve (a regression bound).  ulp = (min_identical, steps): both bf16, at
    least that fraction bit-identical and no element further from the oracle than
    ``steps`` bf16 steps of its row's largest oracle magnitude."""
    g16 = got if got.dtype == torch.bfloat16 else None
    w16 = want if want.dtype == torch.bfloat16 else None
    got = got.double()
    want = want.double()
    if skip_rows is not None and skip_rows.any():
        keep = ~skip_rows
        got, want = got[keep], want[keep]
        g16 = None if g16 is None else g16[keep]
        w16 = None if w16 is None else w16[keep]
    d = (got - want).abs()
    mx = (d.max() / want.abs().max()).item()
    mean = (d.mean() / want.abs().mean()).item()
    exact = (d == 0).double().mean().item()
    msg = (f"{label}: rows {got.shape[0]} max|d|/max|ref|={mx:.3e} mean|d|/mean|ref|={mean:.3e} "
           f"raw max|d|={d.max().item():.4g} max|ref|={want.abs().max().item():.4g} "
           f"bit-identical={exact:.4f}")
    if g16 is not None and w16 is not None:
        u = bf16_ulp_distance(g16, w16)
        row_step = bf16_step(want.abs().max(1, keepdim=True).values)
        rel_step = (d / row_step).max().item()
        msg += (f" elements >1 ulp={int((u > 1).sum())} max|d|/row step={rel_step:.3f}")
    print(msg, flush=True)
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)
    if mean_bound is not None:
        assert mean <= mean_bound, f"{label}: mean rel {mean:.3e} above the regression bound " \
                                   f"{mean_bound:.1e}"
    if ulp is not None:
        assert g16 is not None and w16 is not None, "ulp bounds need bf16 outputs"
        min_identical, steps = ulp
        assert exact >= min_identical, f"{label}: {exact:.4f} bit-identical < {min_identical}"
        assert rel_step <= steps, f"{label}: an element {rel_step:.3f} bf16 steps of its " \
                                  f"row's largest output away (bound {steps})"
    return mx, mean
