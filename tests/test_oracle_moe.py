"""Pins of oracle.moe_cte / oracle.moe_block_tkg / oracle.layer.

* The dense reference flows against a float64 closed form of the per-(token, expert)
  algebra: g = x.Wg + bg, u = x.Wu + bu, g' = min(g, limit), u' = clamp(u, -limit+1,
  limit+1), h = u' * g' * sigmoid(1.702 g'), y = h.Wd + bd, out = sum_k a_k y_k.
* The routed forms against the dense forms (they skip only zero-affinity experts).
"""

import math

import pytest
import torch

from oracle import moe_block_tkg as obt
from oracle import moe_cte as oc
from oracle.layer import RefLayer


def _mini_layer(E=4, H=64, I=32, K=2, limit=7.0, biases=True, seed=0, exp=(118, 122)):
    import pkgload
    pkgload.load()
    from vllm_neuron_amd import synthetic

    shape = synthetic.MoEShape("mini", E, K, H, I, swiglu_limit=limit, biases=biases)
    return synthetic.layer_tensors(shape, seed, exp_range=exp), synthetic


def closed_form(layer, x, aff):
    """float64 per-(token, expert) algebra of the GPT-OSS expert block."""
    xd = x.double()
    gu = layer.gate_up.double()  # [E, H, 2I]
    I = layer.I
    out = torch.zeros(x.shape[0], layer.H, dtype=torch.float64)
    for t in range(x.shape[0]):
        for e in range(layer.E):
            a = float(aff[t, e])
            if a == 0:
                continue
            z = xd[t] @ gu[e]
            if layer.gu_bias is not None:
                z = z + layer.gu_bias[e].double()
            g, u = z[:I], z[I:]
            if layer.limit is not None:
                g = torch.minimum(g, torch.tensor(layer.limit, dtype=torch.float64))
                u = u.clamp(-layer.limit + 1, layer.limit + 1)
                act = g * torch.sigmoid(1.702 * g)
            else:
                act = g * torch.sigmoid(g)
            y = (u * act) @ layer.down[e].double()
            if layer.dn_bias is not None:
                y = y + layer.dn_bias[e].double()
            out[t] += a * y
    return out


def rel_errs(got, want):
    d = (got.double() - want.double()).abs()
    return (d.max() / want.abs().max()).item(), (d.mean() / want.abs().mean()).item()


@pytest.mark.parametrize("limit,biases", [(7.0, True), (None, False)])
def test_decode_dense_vs_closed_form(limit, biases):
    lt, syn = _mini_layer(limit=limit, biases=biases)
    layer = RefLayer(lt)
    x = syn.tokens(3, 5, layer.H)
    out, aff = layer.decode(x)
    want = closed_form(layer, x, aff)
    mx, mean = rel_errs(out.float(), want)
    assert mx < 8e-3 and mean < 3e-3  # one bf16 rounding of the output


@pytest.mark.parametrize("limit,biases", [(7.0, True), (None, False)])
def test_prefill_dense_vs_closed_form(limit, biases):
    lt, syn = _mini_layer(limit=limit, biases=biases)
    layer = RefLayer(lt)
    x = syn.tokens(4, 40, layer.H)
    out, aff = layer.prefill(x)
    want = closed_form(layer, x, aff)
    mx, mean = rel_errs(out, want)
    assert mx < 3e-2 and mean < 1e-2  # bf16 intermediates of the reference flow


def test_routed_forms_match_dense():
    lt, syn = _mini_layer(E=6, K=3, seed=2)
    layer = RefLayer(lt)
    x = syn.tokens(5, 33, layer.H)
    d_out, aff = layer.decode(x)
    r_out = layer.decode_routed(x, aff)
    assert torch.equal(d_out, r_out)
    p_out, aff = layer.prefill(x)
    rp = layer.prefill_routed(x, aff)
    mx, mean = rel_errs(rp, p_out)
    assert mx < 1e-2 and mean < 1e-3
    rows = torch.tensor([0, 7, 32])
    rs = layer.prefill_routed(x, aff, token_rows=rows)
    assert torch.equal(rs, rp[rows])


def test_swiglu_clamp_special_cases():
    # g at the clamp, u at both clamps, very negative g -> -0 product
    g = torch.tensor([7.0, 9.0, -200.0, 0.0], dtype=torch.float32)
    u = torch.tensor([-7.0, 10.0, 3.0, 1.0], dtype=torch.float32)
    gc = g.clamp(max=7.0)
    uc = u.clamp(-6.0, 8.0)
    h = uc * oc.apply_activation(gc, oc.SWISH)
    want = [-6.0 * 7.0 / (1 + math.exp(-1.702 * 7.0)), 8.0 * 7.0 / (1 + math.exp(-1.702 * 7.0)),
            0.0, 0.0]
    assert torch.allclose(h.double(), torch.tensor(want, dtype=torch.float64), rtol=1e-6)
    assert math.copysign(1.0, float(h[2])) == -1.0 or float(h[2]) == 0.0


def test_block_tkg_impl_matches_layer_decode():
    lt, syn = _mini_layer(E=4, K=2, seed=5)
    layer = RefLayer(lt)
    x = syn.tokens(6, 3, layer.H)
    gamma = torch.ones(layer.H)
    out, logits = obt.torch_moe_block_tkg_impl(
        x, gamma, layer.router_w.T, layer.gate_up.reshape(layer.E, layer.H, 2, layer.I),
        layer.down, None, layer.gu_bias.reshape(layer.E, 2, layer.I), layer.dn_bias, 1e-6, 2,
        "SOFTMAX", False, False, "POST_SCALE", oc.SWISH, 7.0, None, 8.0, -6.0)
    xn, _, _, _ = obt.rmsnorm_router(x, gamma, layer.router_w.T, None, 1e-6, 2, "SOFTMAX",
                                     False, False)
    want, _ = layer.decode(xn)
    assert torch.equal(out, want)


def test_lazy_layer_matches_eager():
    """The per-expert lazy dequantization gives the routed forms the same weights."""
    lt, syn = _mini_layer(E=6, K=2, seed=7)
    eager, lazy = RefLayer(lt), RefLayer(lt, lazy=True)
    x = syn.tokens(8, 20, eager.H)
    aff, _ = eager.route(x)
    assert torch.equal(eager.decode_routed(x, aff), lazy.decode_routed(x, aff))
    assert torch.equal(eager.prefill_routed(x, aff), lazy.prefill_routed(x, aff))


def closed_form_pre(layer, x, aff, mode, routed_only=False):
    """float64 algebra of the pre-scaling modes (moe_cte.py:465-495): every expert of every
    token contributes; PRE_SCALE scales the hidden row by the affinity before gate/up,
    PRE_SCALE_DELAYED the activation before down; no weighting after down.  routed_only
    drops the experts a token does not route to (a plausible mistake)."""
    xd = x.double()
    gu = layer.gate_up.double()
    I = layer.I
    out = torch.zeros(x.shape[0], layer.H, dtype=torch.float64)
    lim = torch.tensor(layer.limit, dtype=torch.float64)
    for t in range(x.shape[0]):
        for e in range(layer.E):
            a = float(aff[t, e])
            if routed_only and a == 0:
                continue
            z = ((a * xd[t]) if mode == oc.PRE_SCALE else xd[t]) @ gu[e] + layer.gu_bias[e].double()
            g, u = torch.minimum(z[:I], lim), z[I:].clamp(-layer.limit + 1, layer.limit + 1)
            h = u * g * torch.sigmoid(1.702 * g)
            if mode == oc.PRE_SCALE_DELAYED:
                h = h * a
            out[t] += h @ layer.down[e].double() + layer.dn_bias[e].double()
    return out


@pytest.mark.parametrize("mode", [oc.PRE_SCALE, oc.PRE_SCALE_DELAYED])
def test_prescale_modes_vs_closed_form(mode):
    """The oracle's pre-scaling flows (bf16 affinities, bf16 running sum over all experts)
    against the float64 algebra, with biases large enough that the contributions of the
    experts a token does not route to are a visible share of the output."""
    from oracle import blockwise as obw

    lt, syn = _mini_layer(E=4, K=2, seed=11)
    lt.gate_up_bias = lt.gate_up_bias * 50
    lt.down_bias = lt.down_bias * 50
    layer = RefLayer(lt)
    x = syn.tokens(12, 24, layer.H)
    aff, _ = layer.route(x)
    aff = aff.to(torch.bfloat16)
    aff_m, _, _, _ = obw.build_blockwise_mapping(aff.float(), layer.E, layer.K, 256)
    gu, gb, db = layer._cte_args()
    got = oc.torch_moe_impl(x, aff_m.to(torch.bfloat16), gu, layer.down, gb, db,
                            activation_function=layer.act, expert_affinities_scaling_mode=mode,
                            **layer.clamps)
    assert got.dtype == torch.bfloat16
    want = closed_form_pre(layer, x, aff.float(), mode)
    mx, mean = rel_errs(got.float(), want)
    assert mx < 3e-2 and mean < 1e-2, (mx, mean)
    # the unrouted experts' share is far above that tolerance
    routed = closed_form_pre(layer, x, aff.float(), mode, routed_only=True)
    assert rel_errs(routed, want)[1] > 0.05
