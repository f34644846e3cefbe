"""Oracle pins for the dense MLP flow (oracle.mlp), the gate/up fusion of packed weights,
and the host-side checks of functional.mlp (no GPU needed)."""

import pytest
import torch

from oracle import mlp as om
from oracle import moe_cte as oc


def _dense(seed, T, H, I, bias=True):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, std=1.0: (torch.randn(*s, generator=g) * std).to(torch.bfloat16)  # noqa: E731
    x = r(T, H)
    gw, uw, dw = r(H, I, std=H ** -0.5), r(H, I, std=H ** -0.5), r(I, H, std=I ** -0.5)
    gb, ub, db = (r(1, I, std=0.1), r(1, I, std=0.1), r(1, H, std=0.1)) if bias else (None,) * 3
    return x, gw, uw, dw, gb, ub, db


@pytest.mark.parametrize("act", ["SiLU", "GELU"])
@pytest.mark.parametrize("bias", [True, False])
def test_mlp_flow_is_moe_flow_with_one_expert(act, bias):
    """The dense flow against _torch_moe_impl with E = 1 and affinity 1 (a separate
    restatement of another reference function with the same per-op bf16 results)."""
    T, H, I = 9, 64, 96
    x, gw, uw, dw, gb, ub, db = _dense(1, T, H, I, bias)
    want = om.torch_mlp_impl(x, gw, uw, dw, act, gb, ub, db)
    gu = torch.stack([gw, uw], 1).unsqueeze(0)          # [1, H, 2, I]
    gub = None if gb is None else torch.stack([gb[0], ub[0]], 0).unsqueeze(0)  # [1, 2, I]
    dnb = None if db is None else db.reshape(1, 1, H)
    got = oc.torch_moe_impl(x, torch.ones(T, 1), gu, dw.unsqueeze(0), gub, dnb,
                            activation_function=act)
    assert got.dtype == torch.float32
    d = (got - want.float()).abs()
    # The two flows run their bf16 matmuls through different torch calls (a matmul and
    # an einsum): equal up to the fp32 summation order, i.e. one bf16 step at most.
    assert torch.all(d <= want.float().abs() * 2.0 ** -7 + 1e-6), d.max()
    assert (d == 0).float().mean().item() > 0.95


def test_mlp_flow_closed_form_zero_gate():
    """gate_w = 0: gate = gate_b exactly, so out = (silu(gb) * (x @ up_w + ub)) @ down_w + db,
    evaluated in float64 from the same bf16 operands (one bf16 rounding per op apart)."""
    T, H, I = 7, 64, 32
    x, _, uw, dw, gb, ub, db = _dense(2, T, H, I)
    gw = torch.zeros(H, I, dtype=torch.bfloat16)
    got = om.torch_mlp_impl(x, gw, uw, dw, "SiLU", gb, ub, db).double()
    g = gb.double()
    a = g * torch.sigmoid(g)
    up = x.double() @ uw.double() + ub.double()
    want = (a * up) @ dw.double() + db.double()
    d = (got - want).abs()
    assert (d.max() / want.abs().max()).item() < 2e-2
    assert (d.mean() / want.abs().mean()).item() < 5e-3


def test_mlp_swish_is_silu():
    """mlp.py:278-279 maps Swish to silu (unlike moe_cte's 1.702 form)."""
    v = torch.linspace(-6, 6, 97)
    assert torch.equal(om.activation_fn("Swish")(v), torch.nn.functional.silu(v))
    assert not torch.equal(oc.apply_activation(v, "Swish"), torch.nn.functional.silu(v))


@pytest.mark.parametrize("I,H", [(64, 96), (48, 160), (32, 2880)])
def test_fuse_gate_up_matches_packing_interleaved_rows(I, H):
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd import weights as W

    gb, gs = synthetic.mxfp4_tensor(3, I, H, 100, 140)
    ub, us = synthetic.mxfp4_tensor(4, I, H, 100, 140)
    gq, gsp = W.pack_mxfp4(gb, gs)
    uq, usp = W.pack_mxfp4(ub, us)
    fq, fs = W.fuse_gate_up(gq, gsp, uq, usp)
    rq, rs = W.pack_mxfp4(W.interleave_row_groups(gb[None], ub[None])[0],
                          W.interleave_row_groups(gs[None], us[None])[0])
    assert torch.equal(fq, rq) and torch.equal(fs, rs)
    gc, gs8 = synthetic.mxfp8_tensor(5, I, H)
    uc, us8 = synthetic.mxfp8_tensor(6, I, H)
    g8, gs8p = W.pack_mxfp8(gc, gs8)
    u8, us8p = W.pack_mxfp8(uc, us8)
    f8, fs8 = W.fuse_gate_up(g8, gs8p, u8, us8p)
    r8, rs8 = W.pack_mxfp8(W.interleave_row_groups(gc[None], uc[None])[0],
                           W.interleave_row_groups(gs8[None], us8[None])[0])
    assert torch.equal(f8, r8) and torch.equal(fs8, rs8)


@pytest.mark.parametrize("kw,exc", [
    ({"quantization_type": "NONE"}, NotImplementedError),
    ({"quantization_type": "STATIC"}, NotImplementedError),
    ({"norm_type": "RMS_NORM"}, NotImplementedError),
    ({"fused_add_tensor": torch.zeros(2, 64, dtype=torch.bfloat16)}, NotImplementedError),
    ({"skip_gate": True}, NotImplementedError),
    ({"act_fn": "GELU_Tanh_Approx"}, NotImplementedError),
    ({"gate_up_in_scale": torch.ones(1)}, NotImplementedError),
    ({"gate_w_scale": None}, AssertionError),
])
def test_mlp_host_checks(kw, exc):
    from vllm_neuron_amd.enums import NormType, QuantizationType
    from vllm_neuron_amd.functional import mlp

    args = {"quantization_type": QuantizationType.MX, "norm_type": NormType.NO_NORM,
            "gate_w_scale": torch.zeros(1, 128, dtype=torch.uint8),
            "up_w_scale": torch.zeros(1, 128, dtype=torch.uint8),
            "down_w_scale": torch.zeros(1, 64, dtype=torch.uint8)}
    for k, v in kw.items():
        args[k] = getattr(QuantizationType, v) if k == "quantization_type" else (
            getattr(NormType, v) if k == "norm_type" else v)
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    w = torch.zeros(2, 512, dtype=torch.uint8)
    with pytest.raises(exc):
        mlp(x, w, w, torch.zeros(4, 256, dtype=torch.uint8), **args)
