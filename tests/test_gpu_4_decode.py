"""Decode expert path (router -> moe_tkg) vs the oracle's moe_block_tkg flow (fp32)."""

import pytest
import torch

from moe_helpers import BF16_OUT, build, check_close, check_indices, decode_checked

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gptoss20(dev):
    from vllm_neuron_amd import synthetic

    return build(synthetic.GPT_OSS_20B, 1, dev)


@pytest.mark.parametrize("T", [1, 4, 16, 48, 64])
def test_decode_gptoss20b(dev, gptoss20, T):
    from vllm_neuron_amd import synthetic

    ref, layer, _ = gptoss20
    x = synthetic.tokens(21, T, ref.H)
    got, aff, ties = decode_checked(layer, ref, x, dev)
    want = ref.decode_routed(x, aff)
    check_close(got, want, ties, f"decode 20b T={T}", ulp=BF16_OUT)


@pytest.mark.parametrize("E,T,zipf", [(32, 64, 1.2), (64, 48, 1.5)])
def test_decode_skewed_routing_hot_experts(dev, E, T, zipf):
    """Zipf-skewed routing: the hottest experts hold several 16-token tiles, each tile its
    own work item of the decode kernels."""
    from vllm_neuron_amd import synthetic

    ref, layer, _ = build(synthetic.GPT_OSS_20B, 41, dev, E=E, zipf=zipf)
    x = synthetic.tokens(43, T, ref.H)
    got, aff, ties = decode_checked(layer, ref, x, dev)
    per_expert = (aff != 0).sum(0)
    print(f"tokens per expert: max {int(per_expert.max())}, experts touched "
          f"{int((per_expert > 0).sum())}")
    assert per_expert.max() > 32  # at least three tiles for one expert
    want = ref.decode_routed(x, aff)
    check_close(got, want, ties, f"decode skewed E={E} T={T} zipf={zipf}", ulp=BF16_OUT)


@pytest.mark.parametrize("T", [16, 64])
def test_decode_repeated_calls_and_graph_replays(dev, gptoss20, T):
    """Consecutive calls on one cached workspace, and replays of a captured graph with
    eager work in between, give the same bits as the first eager call."""
    from vllm_neuron_amd import synthetic

    ref, layer, _ = gptoss20
    x = synthetic.tokens(31, T, ref.H).to(dev)
    first = layer.decode(x)
    for _ in range(3):
        assert torch.equal(layer.decode(x), first)
    x2 = synthetic.tokens(32, T, ref.H).to(dev)
    other = layer.decode(x2)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            out = layer.decode(x)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first), f"replay {i}"
        assert torch.equal(layer.decode(x2), other)  # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("E,k,T", [(300, 8, 37), (512, 4, 128)])
def test_decode_wide_expert_counts(dev, E, k, T):
    """Expert counts that are not multiples of 64 and the widest rows of the decode
    front end's top-k (up to 8 logits per lane)."""
    from vllm_neuron_amd import synthetic

    shape = synthetic.MoEShape(f"wide{E}", E, k, 256, 256)
    ref, layer, _ = build(shape, 40 + E, dev, exp=(118, 122))
    x = synthetic.tokens(41, T, ref.H)
    got, aff, ties = decode_checked(layer, ref, x, dev)
    want = ref.decode_routed(x, aff)
    check_close(got, want, ties, f"decode E={E} k={k} T={T}", ulp=BF16_OUT)


@pytest.mark.parametrize("T", [200, 256])
def test_decode_large_batch(dev, gptoss20, T):
    """Batches past the fused front end (standalone router + routing kernels) and with
    more than 8 routed tokens per expert on average (two token tiles per pass)."""
    from vllm_neuron_amd import synthetic

    ref, layer, _ = gptoss20
    x = synthetic.tokens(33, T, ref.H)
    got, aff, ties = decode_checked(layer, ref, x, dev)
    want = ref.decode_routed(x, aff)
    check_close(got, want, ties, f"decode 20b T={T}", ulp=BF16_OUT)


def test_decode_unsaturated_weights(dev):
    from vllm_neuron_amd import synthetic

    ref, layer, _ = build(synthetic.GPT_OSS_20B, 2, dev, E=16, exp=(116, 120))
    x = synthetic.tokens(22, 40, ref.H)
    got, aff, ties = decode_checked(layer, ref, x, dev)
    want = ref.decode_routed(x, aff)
    check_close(got, want, ties, "decode unsaturated", ulp=BF16_OUT)


def test_decode_dense_flow_equals_routed(dev):
    """The dense all-expert flow of the reference on a small layer, end to end."""
    from vllm_neuron_amd import synthetic

    shape = synthetic.MoEShape("mini", 8, 2, 256, 512)
    ref, layer, _ = build(shape, 3, dev, exp=(118, 122))
    x = synthetic.tokens(23, 9, ref.H)
    want, aff = ref.decode(x)
    got = layer.decode(x.to(dev)).cpu()
    check_close(got, want, None, "decode dense mini")


def test_decode_plain_swiglu_fine_grained(dev):
    from vllm_neuron_amd import synthetic

    ref, layer, _ = build(synthetic.FINE_GRAINED, 4, dev, E=32)
    x = synthetic.tokens(24, 8, ref.H)
    got, aff, ties = decode_checked(layer, ref, x, dev)
    want = ref.decode_routed(x, aff)
    check_close(got, want, ties, "decode plain swiglu", ulp=BF16_OUT)


def test_moe_tkg_api_ep_rank_and_no_scale(dev):
    """moe_tkg with global expert ids and rank_id (local slice), NO_SCALE mode."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic

    from oracle import moe_block_tkg as obt

    shape = synthetic.MoEShape("mini", 8, 2, 256, 256)
    ref, layer, _ = build(shape, 5, dev, exp=(118, 122))
    T, E_g = 12, 16
    x = synthetic.tokens(25, T, ref.H)
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(T, E_g, generator=g)
    vals, idx = torch.topk(logits, 2, dim=1)
    aff_full = torch.zeros(T, E_g).scatter_(1, idx, torch.softmax(vals, 1))
    w = layer.w
    got = NF.moe_tkg(x.to(dev), w.gu_q, w.dn_q, aff_full.to(dev), idx.to(torch.int32).to(dev),
                     is_all_expert=False, rank_id=torch.tensor([[1]], device=dev),
                     expert_gate_up_bias=w.gu_bias, expert_down_bias=w.dn_bias,
                     expert_gate_up_weights_scale=w.gu_s, expert_down_weights_scale=w.dn_s,
                     expert_affinities_scaling_mode="NO_SCALE", activation_fn="Swish",
                     gate_clamp_upper_limit=7.0, up_clamp_upper_limit=8.0,
                     up_clamp_lower_limit=-6.0).cpu()
    local = aff_full[:, 8:16]
    gu = ref.gate_up.reshape(8, ref.H, 2, ref.I)
    want = obt.expert_mlp_fp32_routed(x, local, gu, ref.down, ref.gu_bias.reshape(8, 2, ref.I),
                                      ref.dn_bias, hidden_act_fn="Swish",
                                      gate_clamp_upper_limit=7.0, up_clamp_upper_limit=8.0,
                                      up_clamp_lower_limit=-6.0, scale_mode="NO_SCALE",
                                      out_dtype=torch.bfloat16)
    rows = (local != 0).any(1)
    assert torch.all(got[~rows] == 0)
    check_close(got[rows], want[rows], None, "moe_tkg ep rank 1, NO_SCALE")


def test_moe_block_tkg_api(dev):
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic

    from oracle import moe_block_tkg as obt

    ref, layer, _ = build(synthetic.GPT_OSS_20B, 6, dev, E=32)
    T = 16
    x = synthetic.tokens(26, T, ref.H)
    gamma = torch.ones(ref.H)
    w = layer.w
    out, logits = NF.moe_block_tkg(
        x.unsqueeze(0).to(dev), gamma.unsqueeze(0).to(dev), ref.router_w.T.to(dev), w.gu_q, w.dn_q,
        top_k=4, expert_gate_up_weights_scale=w.gu_s, expert_down_weights_scale=w.dn_s,
        expert_gate_up_bias=w.gu_bias, expert_down_bias=w.dn_bias, router_act_fn="SOFTMAX",
        router_pre_norm=False, expert_affinities_scaling_mode="POST_SCALE",
        hidden_act_fn="Swish", gate_clamp_upper_limit=7.0, up_clamp_upper_limit=8.0,
        up_clamp_lower_limit=-6.0)
    xn, logits_r, top, idx = obt.rmsnorm_router(x, gamma, ref.router_w.T, None, 1e-6, 4,
                                                "SOFTMAX", False, False)
    aff = torch.zeros(T, ref.E).scatter_(1, idx, top)
    want = ref.decode_routed(xn, aff)
    assert torch.allclose(logits.cpu(), logits_r, rtol=1e-5, atol=1e-5)
    check_close(out.cpu(), want, None, "moe_block_tkg")


@pytest.mark.parametrize("T,act,pre_norm,renorm,ha", [(64, "SIGMOID", True, True, 2800),
                                                      (40, "SOFTMAX", False, False, None)])
def test_moe_block_tkg_api_norm_and_router_options(dev, T, act, pre_norm, renorm, ha):
    """The one-call block path (RMSNorm with a random gamma over the first ha columns,
    router options, experts) against the oracle's RMSNorm + router and routed layer."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic

    from oracle import moe_block_tkg as obt

    ref, layer, _ = build(synthetic.GPT_OSS_20B, 8, dev, E=32)
    x = synthetic.tokens(28, T, ref.H)
    gamma = 1.0 + 0.1 * torch.randn(ref.H, generator=torch.Generator().manual_seed(3))
    w = layer.w
    rw = ref.router_w.T.contiguous().to(dev)
    args = dict(top_k=4, expert_gate_up_weights_scale=w.gu_s, expert_down_weights_scale=w.dn_s,
                expert_gate_up_bias=w.gu_bias, expert_down_bias=w.dn_bias, router_act_fn=act,
                router_pre_norm=pre_norm, norm_topk_prob=renorm,
                expert_affinities_scaling_mode="POST_SCALE", hidden_act_fn="Swish",
                hidden_actual=ha, **ref.clamps)
    out, logits = NF.moe_block_tkg(x.to(dev), gamma.to(dev), rw, w.gu_q, w.dn_q, **args)
    out2, _ = NF.moe_block_tkg(x.to(dev), gamma.to(dev), rw, w.gu_q, w.dn_q, **args)
    assert torch.equal(out, out2)  # the cached transposed router weights give the same result
    xn, logits_r, top, idx = obt.rmsnorm_router(x, gamma, ref.router_w.T, None, 1e-6, 4, act,
                                                pre_norm, renorm, ha)
    assert torch.allclose(logits.cpu(), logits_r, rtol=1e-4, atol=1e-4)
    aff = torch.zeros(T, ref.E).scatter_(1, idx, top)
    want = ref.decode_routed(xn, aff)
    check_close(out.cpu(), want, None, f"moe_block_tkg {act} pre_norm={pre_norm} ha={ha}")


def test_moe_block_tkg_api_expert_slice(dev):
    """A rank holding 16 of 32 experts (rank_id 1): RMSNorm, router over all 32, local
    ids, experts of the slice."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.weights import MXFP4Experts

    from oracle import moe_block_tkg as obt

    ref, layer, lt = build(synthetic.GPT_OSS_20B, 9, dev, E=32)
    T = 16
    x = synthetic.tokens(29, T, ref.H)
    gamma = torch.ones(ref.H)
    w = MXFP4Experts.from_checkpoint(lt.gate_up_blocks[16:], lt.gate_up_scales[16:],
                                     lt.down_blocks[16:], lt.down_scales[16:],
                                     lt.gate_up_bias[16:], lt.down_bias[16:]).to(dev)
    out, _ = NF.moe_block_tkg(
        x.to(dev), gamma.to(dev), ref.router_w.T.contiguous().to(dev), w.gu_q, w.dn_q,
        rank_id=torch.tensor([1], device=dev), top_k=4, expert_gate_up_weights_scale=w.gu_s,
        expert_down_weights_scale=w.dn_s, expert_gate_up_bias=w.gu_bias,
        expert_down_bias=w.dn_bias, router_act_fn="SOFTMAX", router_pre_norm=False,
        expert_affinities_scaling_mode="POST_SCALE", hidden_act_fn="Swish", **ref.clamps)
    xn, _, top, idx = obt.rmsnorm_router(x, gamma, ref.router_w.T, None, 1e-6, 4, "SOFTMAX",
                                         False, False)
    aff = torch.zeros(T, ref.E).scatter_(1, idx, top)
    aff[:, :16] = 0.0
    want = ref.decode_routed(xn, aff)
    check_close(out.cpu(), want, None, "moe_block_tkg expert slice")


def test_decode_gptoss120b_t64(dev):
    """120B-shaped layer (128 experts) at 64 tokens, every token against the oracle."""
    from vllm_neuron_amd import synthetic

    ref, layer, _ = build(synthetic.GPT_OSS_120B, 7, dev)
    x = synthetic.tokens(27, 64, ref.H)
    got, aff, ties = decode_checked(layer, ref, x, dev)
    want = ref.decode_routed(x, aff)
    check_close(got, want, ties, "decode 120b T=64", ulp=BF16_OUT)


@pytest.mark.parametrize("T", [4, 64])
def test_decode_unaligned_biases(dev, gptoss20, T):
    """Biases that are not 8-byte aligned (a view 2 bytes into its storage) take the
    epilogue's element loads instead of the 8-byte loads issued before the weights
    stream; the arithmetic is the same, so the outputs are bit-identical."""
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.layer import MXFP4MoE

    ref, layer, _ = gptoss20
    w = layer.w
    x = synthetic.tokens(71, T, ref.H).to(dev)
    want = layer.decode(x)

    def shifted(b):
        buf = torch.empty(b.numel() + 1, dtype=b.dtype, device=b.device)
        v = buf[1:].view(b.shape)
        v.copy_(b)
        assert v.data_ptr() % 8 == 2
        return v

    import dataclasses
    w2 = dataclasses.replace(w, gu_bias=shifted(w.gu_bias), dn_bias=shifted(w.dn_bias))
    lay2 = MXFP4MoE(w2, layer.router_w, layer.router_b, layer.top_k, layer.limit)
    got = lay2.decode(x)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
