"""Dense MLP with MX weights (functional.mlp, quantization_type=MX) against the reference's
dense torch flow (oracle.mlp, mlp.py:371-418) on the dequantized weights: MXFP4 and MXFP8,
1 to 1000 tokens, with and without biases and clamps, SiLU / Swish (= silu) / GELU, bf16 and
fp32 outputs.  Bounds: normalized max 2e-2, mean 5e-3 (tests/moe_helpers.check_close)."""

import pytest
import torch

from oracle import mlp as om
from oracle import mxfp4 as o4
from oracle import mxfp8 as o8

from moe_helpers import check_close

pytestmark = pytest.mark.gpu

CASES = [
    # T, H, I, act, bias, clamp, output dtype
    (1, 256, 384, "SiLU", True, False, torch.bfloat16),
    (100, 512, 256, "GELU", False, False, torch.float32),
    (129, 96, 64, "Swish", True, False, torch.bfloat16),
    (1000, 2880, 2880, "SiLU", True, True, torch.bfloat16),
]


def _weights(fmt, seed, rows, K):
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.weights import pack_mxfp4, pack_mxfp8

    if fmt == "mxfp4":
        b, s = synthetic.mxfp4_tensor(seed, rows, K, 118, 122)
        return pack_mxfp4(b, s), o4.dequantize_mxfp4_to_bf16(b, s).reshape(rows, K)
    c, s = synthetic.mxfp8_tensor(seed, rows, K)
    return pack_mxfp8(c, s), o8.dequantize_mxfp8_to_bf16(c, s).reshape(rows, K)


@pytest.mark.parametrize("fmt", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("T,H,I,act,bias,clamp,out_dt", CASES)
def test_mlp_mx(dev, fmt, T, H, I, act, bias, clamp, out_dt):
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.enums import QuantizationType
    from vllm_neuron_amd.functional import mlp

    print(f"mlp {fmt} T={T} H={H} I={I} {act} bias={bias} clamp={clamp} {out_dt}", flush=True)
    (gq, gs), gd = _weights(fmt, 31 + I, I, H)
    (uq, us), ud = _weights(fmt, 37 + I, I, H)
    (dq, ds), dd = _weights(fmt, 41 + H, H, I)
    x = synthetic.normal_bf16(43 + T, (T, H))
    gb = ub = db = None
    if bias:
        gb = synthetic.normal_bf16(47, (1, I), 0.1)
        ub = synthetic.normal_bf16(53, (1, I), 0.1)
        db = synthetic.normal_bf16(59, (1, H), 0.1)
    lim = (None, 7.0, -6.0, 8.0) if clamp else (None,) * 4
    want = om.torch_mlp_impl(x, gd.T.contiguous(), ud.T.contiguous(), dd.T.contiguous(), act,
                             gb, ub, db, lim if clamp else None)
    mv = lambda t: None if t is None else t.to(dev)  # noqa: E731
    got = mlp(x.to(dev), gq.to(dev), uq.to(dev), dq.to(dev), act_fn=act, gate_b=mv(gb),
              up_b=mv(ub), down_b=mv(db), quantization_type=QuantizationType.MX,
              gate_w_scale=gs.to(dev), up_w_scale=us.to(dev), down_w_scale=ds.to(dev),
              output_dtype=out_dt, gate_clamp_lower_limit=lim[0], gate_clamp_upper_limit=lim[1],
              up_clamp_lower_limit=lim[2], up_clamp_upper_limit=lim[3])
    assert got.dtype == out_dt and got.shape == (T, H)
    check_close(got.float().cpu(), want.float(), label=f"mlp {fmt} T={T} {act}")


def test_mlp_mx_weights_cached_and_updated(dev):
    """The fused gate_up is kept per weight version: an in-place update of up_w changes
    the result on the next call."""
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.enums import QuantizationType
    from vllm_neuron_amd.functional import mlp

    H = I = 256
    (gq, gs), gd = _weights("mxfp4", 61, I, H)
    (uq, us), ud = _weights("mxfp4", 67, I, H)
    (dq, ds), dd = _weights("mxfp4", 71, H, I)
    x = synthetic.normal_bf16(73, (16, H))
    args = [t.to(dev) for t in (gq, uq, dq, gs, us, ds)]
    gq_d, uq_d, dq_d, gs_d, us_d, ds_d = args
    run = lambda: mlp(x.to(dev), gq_d, uq_d, dq_d, quantization_type=QuantizationType.MX,  # noqa: E731
                      gate_w_scale=gs_d, up_w_scale=us_d, down_w_scale=ds_d).float().cpu()
    a = run()
    check_close(a, om.torch_mlp_impl(x, gd.T.contiguous(), ud.T.contiguous(),
                                     dd.T.contiguous()).float(), label="mlp before update")
    # new codes under the same scales: the dense reference dequantizes them with up's scales
    from vllm_neuron_amd.weights import unpack_mxfp4
    (uq2, _), _ = _weights("mxfp4", 79, I, H)
    b2, s_up = unpack_mxfp4(uq2, us)
    ud2 = o4.dequantize_mxfp4_to_bf16(b2, s_up).reshape(I, H)
    uq_d.copy_(uq2.to(dev))
    b = run()
    check_close(b, om.torch_mlp_impl(x, gd.T.contiguous(), ud2.T.contiguous(),
                                     dd.T.contiguous()).float(), label="mlp after update")
    assert not torch.equal(a, b)


def test_mlp_mx_graph_replays(dev):
    """The dense MLP (mapping, tile order, both GEMMs, combine) captured in a HIP graph after
    one eager call: every replay, with eager work and synchronizations between them, equals
    the eager result for its input."""
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.enums import QuantizationType
    from vllm_neuron_amd.functional import mlp

    T, H, I = 200, 512, 384
    (gq, gs), _ = _weights("mxfp4", 83, I, H)
    (uq, us), _ = _weights("mxfp4", 89, I, H)
    (dq, ds), _ = _weights("mxfp4", 97, H, I)
    w = [t.to(dev) for t in (gq, uq, dq, gs, us, ds)]
    gb = synthetic.normal_bf16(101, (1, I), 0.1).to(dev)
    run = lambda xx: mlp(xx, w[0], w[1], w[2], quantization_type=QuantizationType.MX,  # noqa: E731
                         gate_w_scale=w[3], up_w_scale=w[4], down_w_scale=w[5], gate_b=gb)
    xs = [synthetic.normal_bf16(103 + i, (T, H)).to(dev) for i in range(3)]
    eager = [run(x).clone() for x in xs]
    torch.cuda.synchronize()
    static_x = xs[0].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run(static_x)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_out = run(static_x)
    for rep in range(2):
        for i, x in enumerate(xs):
            static_x.copy_(x)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(static_out, eager[i]), (rep, i)
            other = run(xs[(i + 1) % 3])  # eager work between replays
            torch.cuda.synchronize()
            assert torch.equal(other, eager[(i + 1) % 3])
