"""Pins of the oracle's RMSNorm and norm + router functions against float64 closed forms.

* oracle.router.rms_norm          (router.py:680-687)
* oracle.moe_block_tkg.rmsnorm_router (moe_block_tkg.py:120-204)
* oracle.rmsnorm_router_topk      (rmsnorm_router_topk_tkg.py:214-279)
* oracle.router with computation_dtype float16 / bfloat16 (router.py:414-503)

Each closed form is written per element from the formulas (float64 sums, one rounding to
the output dtype), never by calling the oracle's own expression.  The inputs make every
term matter: activations small enough that eps is half the denominator, a random gamma,
non-zero columns past hidden_actual, logits spread far apart (no near-ties at the top-k
boundary unless a test builds them), and very negative logits for the +1e-20 of the
renormalization.
"""

import math

import pytest
import torch

from oracle import moe_block_tkg as obt
from oracle import rmsnorm_router_topk as ort
from oracle import router as orr


def _ulp(v: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
    """Spacing of dt at |v| (float64), subnormals included."""
    info = torch.finfo(dt)
    mant = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}[dt]
    a = v.abs().double().clamp(min=info.smallest_normal)
    return torch.pow(2.0, torch.floor(torch.log2(a)) - mant)


def _assert_rounded(got: torch.Tensor, exact: torch.Tensor, dt: torch.dtype, slack=2e-6,
                    min_exact=0.99):
    """got (dtype dt) is exact rounded to dt, up to fp32 noise in the computation: within
    half an ulp plus slack*|exact|, and bit-identical to the rounded exact value almost
    everywhere."""
    assert got.dtype == dt
    g = got.double()
    err = (g - exact).abs()
    bound = 0.5 * _ulp(exact, dt) + slack * exact.abs()
    assert bool((err <= bound).all()), float((err - bound).max())
    same = (got == exact.to(dt)).double().mean().item()
    assert same >= min_exact, same


def _x(T, H, seed, std=1e-3):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(T, H, generator=g, dtype=torch.float64) * std).to(torch.bfloat16)


def _gamma(H, seed):
    g = torch.Generator().manual_seed(seed)
    return (0.5 + torch.rand(H, generator=g, dtype=torch.float64)).to(torch.float32)


def _closed_norm(x, gamma, eps, sum_cols, divisor, zero_from=None):
    """float64: gamma_j * x_j / sqrt(sum_{i < sum_cols} x_i^2 / divisor + eps)."""
    T, H = x.shape
    out = torch.zeros(T, H, dtype=torch.float64)
    for t in range(T):
        ss = sum(float(x[t, i]) ** 2 for i in range(sum_cols))
        inv = 1.0 / math.sqrt(ss / divisor + eps)
        for j in range(H):
            if zero_from is not None and j >= zero_from:
                continue
            out[t, j] = float(gamma[j]) * float(x[t, j]) * inv
    return out


def test_rms_norm_closed_form():
    T, H, eps = 6, 96, 1e-6
    x, gm = _x(T, H, 1), _gamma(H, 2)
    got = orr.rms_norm(x, gm, eps)
    want = _closed_norm(x, gm, eps, H, H)
    _assert_rounded(got, want, torch.bfloat16)


@pytest.mark.parametrize("ha", [80, 96])
def test_block_rmsnorm_closed_form(ha):
    T, H, E, k, eps = 5, 96, 8, 3, 1e-6
    x, gm = _x(T, H, 3), _gamma(H, 4)
    g = torch.Generator().manual_seed(5)
    w = torch.randn(H, E, generator=g).to(torch.bfloat16)
    xn, logits, _, _ = obt.rmsnorm_router(x, gm.unsqueeze(0), w, None, eps, k, "SOFTMAX", False,
                                          False, hidden_actual=ha)
    want = _closed_norm(x, gm, eps, ha, ha, zero_from=ha)
    _assert_rounded(xn, want, torch.bfloat16)
    assert bool((xn[:, ha:] == 0).all())


def _closed_logits(xn, w_he, bias):
    T, E = xn.shape[0], w_he.shape[1]
    out = torch.zeros(T, E, dtype=torch.float64)
    for t in range(T):
        for e in range(E):
            s = sum(float(xn[t, h]) * float(w_he[h, e]) for h in range(xn.shape[1]))
            out[t, e] = s + (float(bias.reshape(-1)[e]) if bias is not None else 0.0)
    return out


def _brute_route(logits, k, fn, pre_norm, renorm):
    """float64 brute force of moe_block_tkg.py:166-204 for one row (list of floats)."""
    E = len(logits)
    if pre_norm:
        if fn == "SOFTMAX":
            m = max(logits)
            ex = [math.exp(v - m) for v in logits]
            score = [v / sum(ex) for v in ex]
        else:
            score = [1.0 / (1.0 + math.exp(-v)) for v in logits]
        order = sorted(range(E), key=lambda e: (-score[e], e))[:k]
        vals = [score[e] for e in order]
    else:
        order = sorted(range(E), key=lambda e: (-logits[e], e))[:k]
        sel = [logits[e] for e in order]
        if fn == "SOFTMAX":
            m = max(sel)
            ex = [math.exp(v - m) for v in sel]
            vals = [v / sum(ex) for v in ex]
        else:
            vals = [1.0 / (1.0 + math.exp(-v)) for v in sel]
    if renorm:
        s = sum(vals) + 1e-20
        vals = [v / s for v in vals]
    return order, vals


@pytest.mark.parametrize("fn", ["SOFTMAX", "SIGMOID"])
@pytest.mark.parametrize("pre_norm,renorm", [(False, False), (False, True), (True, False),
                                             (True, True)])
def test_block_router_brute_force(fn, pre_norm, renorm):
    T, H, E, k, eps = 6, 48, 10, 3, 1e-6
    x = _x(T, H, 6, std=1.0)
    gm = _gamma(H, 7)
    g = torch.Generator().manual_seed(8)
    w = torch.randn(H, E, generator=g).to(torch.bfloat16)
    b = (torch.randn(1, E, generator=g) * 0.5).to(torch.bfloat16)
    xn, logits, top, idx = obt.rmsnorm_router(x, gm, w, b, eps, k, fn, pre_norm, renorm,
                                              hidden_actual=40)
    want_logits = _closed_logits(xn, w, b)
    assert torch.allclose(logits.double(), want_logits, rtol=1e-5, atol=1e-5)
    for t in range(T):
        row = [float(v) for v in want_logits[t]]
        srt = sorted(row, reverse=True)
        assert srt[k - 1] - srt[k] > 1e-3  # tie-free at the boundary
        order, vals = _brute_route(row, k, fn, pre_norm, renorm)
        assert [int(i) for i in idx[t]] == order
        assert torch.allclose(top[t].double(), torch.tensor(vals, dtype=torch.float64),
                              rtol=2e-5, atol=1e-30)


def test_block_router_renorm_epsilon():
    """Sigmoid scores near e^-60: the +1e-20 of the renormalization dominates their sum."""
    T, H, E, k = 3, 32, 6, 2
    x = _x(T, H, 9, std=1.0)
    w = torch.zeros(H, E, dtype=torch.bfloat16)
    b = torch.tensor([[-60.0, -61.0, -62.0, -63.0, -64.0, -65.0]], dtype=torch.bfloat16)
    _, logits, top, idx = obt.rmsnorm_router(x, torch.ones(H), w, b, 1e-6, k, "SIGMOID", True,
                                             True)
    for t in range(T):
        order, vals = _brute_route([float(v) for v in logits[t]], k, "SIGMOID", True, True)
        assert [int(i) for i in idx[t]] == order == [0, 1]
        assert torch.allclose(top[t].double(), torch.tensor(vals, dtype=torch.float64),
                              rtol=1e-5)
        assert float(top[t].sum()) < 1e-4  # without the epsilon it would be 1


@pytest.mark.parametrize("mm", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("ha", [None, 200])
@pytest.mark.parametrize("fn", ["SOFTMAX", "SIGMOID"])
def test_rmsnorm_router_topk_closed_form(mm, ha, fn):
    B, S, H, E, k, eps = 1, 5, 256, 12, 4, 1e-6
    x = _x(B * S, H, 10).reshape(B, S, H)
    gm = _gamma(H, 11)
    g = torch.Generator().manual_seed(12)
    w = (torch.randn(H, E, generator=g) * 2.0).to(torch.float16)
    b = (torch.randn(1, E, generator=g)).to(torch.float16)
    norm, idx, aff, logits = ort.rmsnorm_router_topk(x, gm.unsqueeze(0), w, b, eps, k, ha, mm, fn)
    # norm: every column normalized, mean square over all H divided by hidden_actual
    want = _closed_norm(x.reshape(-1, H), gm, eps, H, H if ha is None else ha)
    _assert_rounded(norm, want, mm)
    # logits from the (cast) operands in float64
    want_l = _closed_logits(norm, w.to(mm), b.to(mm))
    assert torch.allclose(logits.double(), want_l, rtol=1e-5, atol=1e-4)
    for t in range(B * S):
        row = [float(v) for v in want_l[t]]
        srt = sorted(row, reverse=True)
        assert srt[k - 1] - srt[k] > 1e-3
        order, vals = _brute_route(row, k, fn, False, False)
        assert [int(i) for i in idx[t]] == order
        exact = torch.zeros(E, dtype=torch.float64)
        exact[order] = torch.tensor(vals, dtype=torch.float64)
        _assert_rounded(aff[t], exact, torch.bfloat16, slack=1e-5, min_exact=0.9)


@pytest.mark.parametrize("cdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("order", [orr.PRENORM_LINEAR_TOPK_ACT_SCATTER,
                                   orr.PRENORM_LINEAR_ACT_TOPK_RENORM_SCATTER])
def test_router_half_precision_closed_form(cdt, order):
    """router.py:414-503 in a 16-bit computation dtype: operands cast, the bias added to
    the fp32 sum, one rounding of the logit; each activation, sum and quotient rounded."""
    T, H, E, k = 12, 64, 16, 4
    g = torch.Generator().manual_seed(13)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = (torch.randn(E, H, generator=g) * 0.5).to(torch.float16)
    b = torch.randn(E, generator=g).to(torch.float16)
    aff, logits = orr.router(x, w.T, k, b, "softmax", return_logits=True, computation_dtype=cdt,
                             router_computation_order=order)
    assert aff.dtype == cdt and logits.dtype == cdt
    exact = _closed_logits(x.to(cdt), w.T.to(cdt), b.to(cdt))
    _assert_rounded(logits, exact, cdt, min_exact=0.98)
    for t in range(T):
        lv = [float(v) for v in logits[t]]
        if order == orr.PRENORM_LINEAR_TOPK_ACT_SCATTER:
            srt = sorted(lv, reverse=True)
            if srt[k - 1] == srt[k]:
                continue  # an exact tie in cdt: torch.topk's choice is implementation-defined
            sel = sorted(range(E), key=lambda e: (-lv[e], e))[:k]
            m = max(lv[e] for e in sel)
            ex = [math.exp(lv[e] - m) for e in sel]
            want = torch.zeros(E, dtype=torch.float64)
            want[sel] = torch.tensor([v / sum(ex) for v in ex], dtype=torch.float64)
            _assert_rounded(aff[t], want, cdt, slack=1e-6, min_exact=0.75)
        else:
            m = max(lv)
            ex = [math.exp(v - m) for v in lv]
            probs = [float(torch.tensor(v / sum(ex), dtype=torch.float64).to(cdt)) for v in ex]
            srt = sorted(probs, reverse=True)
            if srt[k - 1] == srt[k]:
                continue
            sel = sorted(range(E), key=lambda e: (-probs[e], e))[:k]
            s = float(torch.tensor(sum(probs[e] for e in sel), dtype=torch.float64).to(cdt))
            want = torch.zeros(E, dtype=torch.float64)
            want[sel] = torch.tensor([probs[e] / s for e in sel], dtype=torch.float64)
            _assert_rounded(aff[t], want, cdt, slack=1e-3, min_exact=0.5)
