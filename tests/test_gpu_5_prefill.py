"""Prefill expert path (router -> blockwise mapping -> moe_cte) vs the oracle's
moe_cte torch flow (bf16 intermediates)."""

import pytest
import torch

from moe_helpers import BF16_OUT, PREFILL_FP32_MEAN, build, check_close, routing_agreement

pytestmark = pytest.mark.gpu


def test_prefill_dense_flow_mini(dev):
    from vllm_neuron_amd import synthetic

    shape = synthetic.MoEShape("mini", 8, 2, 256, 512)
    ref, layer, _ = build(shape, 31, dev, exp=(118, 122))
    x = synthetic.tokens(31, 300, ref.H)
    aff, ties = routing_agreement(layer, ref, x, dev)
    want, _ = ref.prefill(x, aff)
    got = layer.prefill(x.to(dev)).cpu()
    check_close(got, want, ties, "prefill dense mini")


@pytest.mark.parametrize("T,zipf", [(512, None), (4096, None), (4096, 1.2)])
def test_prefill_gptoss20b(dev, T, zipf):
    from vllm_neuron_amd import synthetic

    ref, layer, _ = build(synthetic.GPT_OSS_20B, 32 if zipf is None else 33, dev, zipf=zipf)
    x = synthetic.tokens(32, T, ref.H)
    aff, ties = routing_agreement(layer, ref, x, dev)
    xd = x.to(dev)
    got32 = layer.prefill(xd, output_dtype=torch.float32).cpu()
    got16 = layer.prefill(xd).cpu()
    want = ref.prefill_routed(x, aff)  # every row
    check_close(got32, want, ties, f"prefill 20b T={T} zipf={zipf} fp32",
                mean_bound=PREFILL_FP32_MEAN)
    check_close(got16, want.to(torch.bfloat16), ties, f"prefill 20b T={T} zipf={zipf} bf16",
                ulp=BF16_OUT)


def test_prefill_unsaturated(dev):
    from vllm_neuron_amd import synthetic

    ref, layer, _ = build(synthetic.GPT_OSS_20B, 34, dev, E=16, exp=(116, 120))
    x = synthetic.tokens(34, 700, ref.H)
    aff, ties = routing_agreement(layer, ref, x, dev)
    got = layer.prefill(x.to(dev)).cpu()
    rows = torch.arange(0, 700, 7)
    want = ref.prefill_routed(x, aff, token_rows=rows)
    check_close(got[rows], want, ties[rows], "prefill unsaturated")


def test_prefill_plain_swiglu_fine_grained(dev):
    from vllm_neuron_amd import synthetic

    ref, layer, _ = build(synthetic.FINE_GRAINED, 35, dev, E=32, zipf=1.0)
    x = synthetic.tokens(35, 512, ref.H)
    aff, ties = routing_agreement(layer, ref, x, dev)
    got = layer.prefill(x.to(dev)).cpu()
    rows = torch.arange(0, 512, 16)
    want = ref.prefill_routed(x, aff, token_rows=rows)
    check_close(got[rows], want, ties[rows], "prefill plain swiglu")


def test_moe_cte_api_padding_and_skip_token(dev):
    """moe_cte through the reference call pattern with a padding mask; padded tokens
    keep their slots but contribute with zero affinity."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic

    from oracle import blockwise as ob
    from oracle import moe_cte as oc

    shape = synthetic.MoEShape("mini", 8, 2, 256, 256)
    ref, layer, _ = build(shape, 36, dev, exp=(118, 122))
    T = 200
    x = synthetic.tokens(36, T, ref.H)
    aff, ties = routing_agreement(layer, ref, x, dev)
    assert not ties.any()
    pm = torch.arange(T) < 150
    am_g, tp, b2e, cond = NF.build_blockwise_mapping(aff.to(dev), 8, 2, 256, padding_mask=pm.to(dev))
    w = layer.w
    got = NF.moe_cte(x.to(dev), am_g, w.gu_q, w.dn_q, tp, b2e, 256, conditions=cond,
                     gate_and_up_proj_bias=w.gu_bias, down_proj_bias=w.dn_bias,
                     gate_up_proj_scale=w.gu_s, down_proj_scale=w.dn_s,
                     activation_function="Swish", skip_token=True,
                     expert_affinities_scaling_mode="POST_SCALE", gate_clamp_upper_limit=7.0,
                     up_clamp_upper_limit=8.0, up_clamp_lower_limit=-6.0).cpu()
    am_r, _, _, _ = ob.build_blockwise_mapping(aff, 8, 2, 256, padding_mask=pm)
    gu, gb, db = ref._cte_args()
    want = oc.torch_moe_impl(x, am_r, gu, ref.down, gb, db, gate_clamp_upper_limit=7.0,
                             up_clamp_upper_limit=8.0, up_clamp_lower_limit=-6.0,
                             activation_function="Swish")
    assert torch.all(got[150:] == 0)
    check_close(got[:150], want[:150], None, "moe_cte padding mask")


@pytest.mark.parametrize("act", ["GELU", "SiLU"])
def test_moe_cte_and_tkg_other_activations(dev, act):
    """The expert MLP's other activations, unclamped: prefill (moe_cte) and decode
    (moe_tkg) through the reference call pattern against the oracle's flows."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic

    from oracle import blockwise as ob
    from oracle import moe_block_tkg as obt
    from oracle import moe_cte as oc

    shape = synthetic.MoEShape("mini", 8, 2, 256, 256)
    ref, layer, _ = build(shape, 61, dev, exp=(118, 122))
    T = 160
    x = synthetic.tokens(61, T, ref.H)
    aff, _ = routing_agreement(layer, ref, x, dev)
    w = layer.w
    am_g, tp, b2e, cond = NF.build_blockwise_mapping(aff.to(dev), 8, 2, 256)
    got = NF.moe_cte(x.to(dev), am_g, w.gu_q, w.dn_q, tp, b2e, 256, conditions=cond,
                     gate_and_up_proj_bias=w.gu_bias, down_proj_bias=w.dn_bias,
                     gate_up_proj_scale=w.gu_s, down_proj_scale=w.dn_s,
                     activation_function=act, skip_token=True,
                     expert_affinities_scaling_mode="POST_SCALE").cpu()
    am_r, _, _, _ = ob.build_blockwise_mapping(aff, 8, 2, 256)
    gu, gb, db = ref._cte_args()
    want = oc.torch_moe_impl(x, am_r, gu, ref.down, gb, db, activation_function=act)
    check_close(got, want, None, f"moe_cte {act}")

    xd, aff_d = x[:12], aff[:12]
    idx = torch.topk(aff_d, 2, dim=1).indices.to(torch.int32)
    got = NF.moe_tkg(xd.to(dev), w.gu_q, w.dn_q, aff_d.to(dev), idx.to(dev), is_all_expert=False,
                     expert_gate_up_bias=w.gu_bias, expert_down_bias=w.dn_bias,
                     expert_gate_up_weights_scale=w.gu_s, expert_down_weights_scale=w.dn_s,
                     expert_affinities_scaling_mode="POST_SCALE", activation_fn=act).cpu()
    gu4 = ref.gate_up.reshape(8, ref.H, 2, ref.I)
    want = obt.expert_mlp_fp32_routed(xd, aff_d, gu4, ref.down, ref.gu_bias.reshape(8, 2, ref.I),
                                      ref.dn_bias, hidden_act_fn=act, scale_mode="POST_SCALE",
                                      out_dtype=torch.bfloat16)
    check_close(got, want, None, f"moe_tkg {act}")


@pytest.mark.parametrize("T", [1, 3, 17])
def test_prefill_tiny_batches(dev, T):
    """Prefill of a handful of tokens: every M-tile a light one (1-2 subtiles), most of the
    mapping's blocks empty."""
    from vllm_neuron_amd import synthetic

    shape = synthetic.MoEShape("mini", 8, 2, 256, 256)
    ref, layer, _ = build(shape, 71, dev, exp=(118, 122))
    x = synthetic.tokens(71 + T, T, ref.H)
    aff, ties = routing_agreement(layer, ref, x, dev)
    got = layer.prefill(x.to(dev), output_dtype=torch.float32).cpu()
    want, _ = ref.prefill(x, aff)
    check_close(got, want, ties, f"prefill T={T}")


def test_prefill_and_decode_partial_chunks(dev):
    """K below one 128-wide chunk (gate_up, H = 96) and a partial last chunk (down,
    I = 160); 6 row groups of H leave a partial scale quad."""
    from vllm_neuron_amd import synthetic

    shape = synthetic.MoEShape("smallk", 8, 2, 96, 160)
    ref, layer, _ = build(shape, 51, dev, exp=(118, 122))
    x = synthetic.tokens(52, 70, ref.H)
    aff, ties = routing_agreement(layer, ref, x, dev)
    got = layer.prefill(x.to(dev), output_dtype=torch.float32).cpu()
    want, _ = ref.prefill(x, aff)
    check_close(got, want, ties, "prefill small K")
    got = layer.decode(x.to(dev)).cpu()
    want = ref.decode_routed(x, aff)
    check_close(got, want, ties, "decode small K")


@pytest.mark.parametrize("block", [128, 384, 512, 1024])
def test_moe_cte_block_sizes(dev, block):
    """moe_cte at block sizes whose M-tiles the gate_up GEMM schedules in groups of 1,
    1, 4 and 8 (block / 128 tiles, the largest power of two dividing it, at most 16)."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic

    from oracle import blockwise as ob
    from oracle import moe_cte as oc

    shape = synthetic.MoEShape("mini", 8, 2, 256, 256)
    ref, layer, _ = build(shape, 37, dev, exp=(118, 122))
    T = 300
    x = synthetic.tokens(37, T, ref.H)
    aff, ties = routing_agreement(layer, ref, x, dev)
    am_g, tp, b2e, cond = NF.build_blockwise_mapping(aff.to(dev), 8, 2, block)
    w = layer.w
    got = NF.moe_cte(x.to(dev), am_g, w.gu_q, w.dn_q, tp, b2e, block, conditions=cond,
                     gate_and_up_proj_bias=w.gu_bias, down_proj_bias=w.dn_bias,
                     gate_up_proj_scale=w.gu_s, down_proj_scale=w.dn_s,
                     activation_function="Swish", skip_token=True,
                     expert_affinities_scaling_mode="POST_SCALE",
                     gate_clamp_upper_limit=7.0, up_clamp_upper_limit=7.0,
                     up_clamp_lower_limit=-7.0).cpu()
    am_r, _, _, _ = ob.build_blockwise_mapping(aff, 8, 2, block)
    gu, gb, db = ref._cte_args()
    want = oc.torch_moe_impl(x, am_r, gu, ref.down, gb, db, gate_clamp_upper_limit=7.0,
                             up_clamp_upper_limit=7.0, up_clamp_lower_limit=-7.0,
                             activation_function="Swish")
    check_close(got, want, ties, f"moe_cte block {block}")


@pytest.mark.parametrize("mode", ["PRE_SCALE", "PRE_SCALE_DELAYED"])
@pytest.mark.parametrize("biases", [True, False])
def test_moe_cte_prescale_modes(dev, mode, biases):
    """moe_cte's pre-scaling modes against the oracle's dense torch flow (bf16 affinities,
    the bf16 running sum over every expert, moe_cte.py:465-579).  Biases are scaled up so
    that the experts a token does not route to (its y_e(0), or the down bias) are a
    visible share of the output."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.weights import MXFP4Experts

    from oracle import blockwise as ob
    from oracle import moe_cte as oc
    from oracle.layer import RefLayer

    shape = synthetic.MoEShape("mini", 8, 2, 256, 512, biases=biases)
    lt = synthetic.layer_tensors(shape, 37, exp_range=(118, 122))
    if biases:
        lt.gate_up_bias = (lt.gate_up_bias.float() * 20).to(torch.bfloat16)
        lt.down_bias = (lt.down_bias.float() * 20).to(torch.bfloat16)
    ref = RefLayer(lt)
    w = MXFP4Experts.from_checkpoint(lt.gate_up_blocks, lt.gate_up_scales, lt.down_blocks,
                                     lt.down_scales, lt.gate_up_bias, lt.down_bias).to(dev)
    T = 300
    x = synthetic.tokens(37, T, ref.H)
    aff, _ = ref.route(x)
    aff16 = aff.to(torch.bfloat16)
    am_g, tp, b2e, cond = NF.build_blockwise_mapping(aff16.float().to(dev), 8, 2, 256)
    got = NF.moe_cte(x.to(dev), am_g, w.gu_q, w.dn_q, tp, b2e, 256, conditions=cond,
                     gate_and_up_proj_bias=w.gu_bias, down_proj_bias=w.dn_bias,
                     gate_up_proj_scale=w.gu_s, down_proj_scale=w.dn_s,
                     activation_function="Swish", expert_affinities_scaling_mode=mode,
                     gate_clamp_upper_limit=7.0, up_clamp_upper_limit=8.0,
                     up_clamp_lower_limit=-6.0).cpu()
    am_r, _, _, _ = ob.build_blockwise_mapping(aff16.float(), 8, 2, 256)
    gu, gb, db = ref._cte_args()
    want = oc.torch_moe_impl(x, am_r.to(torch.bfloat16), gu, ref.down, gb, db,
                             gate_clamp_upper_limit=7.0, up_clamp_upper_limit=8.0,
                             up_clamp_lower_limit=-6.0, activation_function="Swish",
                             expert_affinities_scaling_mode=mode)
    assert got.dtype == torch.bfloat16 and want.dtype == torch.bfloat16
    check_close(got.float(), want.float(), None, f"moe_cte {mode} biases={biases}")


@pytest.mark.parametrize("biases", [True, False])
def test_moe_cte_no_scale(dev, biases):
    """NO_SCALE against the oracle's dense torch flow: every expert's output for every token
    added unscaled in bf16 (moe_cte.py:518-579); the caller's (routed) mapping is not used."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.weights import MXFP4Experts

    from oracle import moe_cte as oc
    from oracle.layer import RefLayer

    shape = synthetic.MoEShape("mini", 8, 2, 256, 512, biases=biases)
    lt = synthetic.layer_tensors(shape, 38, exp_range=(118, 122))
    ref = RefLayer(lt)
    w = MXFP4Experts.from_checkpoint(lt.gate_up_blocks, lt.gate_up_scales, lt.down_blocks,
                                     lt.down_scales, lt.gate_up_bias, lt.down_bias).to(dev)
    T = 150
    x = synthetic.tokens(38, T, ref.H)
    aff, _ = ref.route(x)
    am_g, tp, b2e, cond = NF.build_blockwise_mapping(aff.to(dev), 8, 2, 256)
    got = NF.moe_cte(x.to(dev), am_g, w.gu_q, w.dn_q, tp, b2e, 256, conditions=cond,
                     gate_and_up_proj_bias=w.gu_bias, down_proj_bias=w.dn_bias,
                     gate_up_proj_scale=w.gu_s, down_proj_scale=w.dn_s,
                     activation_function="Swish", expert_affinities_scaling_mode="NO_SCALE",
                     gate_clamp_upper_limit=7.0, up_clamp_upper_limit=8.0,
                     up_clamp_lower_limit=-6.0).cpu()
    gu, gb, db = ref._cte_args()
    want = oc.torch_moe_impl(x, aff.reshape(-1, 1), gu, ref.down, gb, db,
                             gate_clamp_upper_limit=7.0, up_clamp_upper_limit=8.0,
                             up_clamp_lower_limit=-6.0, activation_function="Swish",
                             expert_affinities_scaling_mode="NO_SCALE")
    assert got.dtype == torch.bfloat16 and want.dtype == torch.bfloat16
    check_close(got.float(), want.float(), None, f"moe_cte NO_SCALE biases={biases}")
    # the same output whatever the routing: an empty mapping gives it too
    zero = torch.zeros_like(aff)
    am0, tp0, b2e0, _ = NF.build_blockwise_mapping(zero.to(dev), 8, 2, 256)
    got0 = NF.moe_cte(x.to(dev), am0, w.gu_q, w.dn_q, tp0, b2e0, 256,
                      gate_and_up_proj_bias=w.gu_bias, down_proj_bias=w.dn_bias,
                      gate_up_proj_scale=w.gu_s, down_proj_scale=w.dn_s,
                      activation_function="Swish", expert_affinities_scaling_mode="NO_SCALE",
                      gate_clamp_upper_limit=7.0, up_clamp_upper_limit=8.0,
                      up_clamp_lower_limit=-6.0).cpu()
    assert torch.equal(got0.view(torch.int16), got.view(torch.int16))


def test_moe_cte_out_of_range_expert_block_is_empty(dev):
    """A block_to_expert entry outside [0, E) (the reference would raise IndexError on its
    weights) computes nothing: its slots add no term, every other block is unchanged."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic

    from oracle import blockwise as ob
    from oracle import moe_cte as oc

    shape = synthetic.MoEShape("mini", 8, 2, 256, 256)
    ref, layer, _ = build(shape, 38, dev, exp=(118, 122))
    T = 200
    x = synthetic.tokens(38, T, ref.H)
    aff, ties = routing_agreement(layer, ref, x, dev)
    am_g, tp, b2e, cond = NF.build_blockwise_mapping(aff.to(dev), 8, 2, 256)
    b2e_h = b2e.cpu()
    first = int(b2e_h[0])  # block 0 holds expert b2e[0]'s first tokens
    bad = b2e.clone()
    bad[0] = 8 + 3
    w = layer.w
    got = NF.moe_cte(x.to(dev), am_g, w.gu_q, w.dn_q, tp, bad, 256,
                     gate_and_up_proj_bias=w.gu_bias, down_proj_bias=w.dn_bias,
                     gate_up_proj_scale=w.gu_s, down_proj_scale=w.dn_s,
                     activation_function="Swish", gate_clamp_upper_limit=7.0,
                     up_clamp_upper_limit=8.0, up_clamp_lower_limit=-6.0).cpu()
    dropped = tp.cpu()[:256]
    dropped = dropped[dropped >= 0]
    aff_cut = aff.clone()
    aff_cut[dropped, first] = 0.0
    am_r, _, _, _ = ob.build_blockwise_mapping(aff, 8, 2, 256)
    am_cut = aff_cut.reshape(-1, 1)
    gu, gb, db = ref._cte_args()
    want = oc.torch_moe_impl(x, am_cut, gu, ref.down, gb, db, gate_clamp_upper_limit=7.0,
                             up_clamp_upper_limit=8.0, up_clamp_lower_limit=-6.0,
                             activation_function="Swish")
    assert len(dropped) > 0
    check_close(got, want, ties, "moe_cte block with out-of-range expert")


def _mxfp8_experts(seed, E, H, I):
    """Random MXFP8 experts: packed GPU tensors (biases [E, 2, I] / [E, H]) and the oracle's
    bf16 [E, H, 2, I] gate_up and [E, I, H] down weights, biases [E, 2, I] / [E, 1, H]."""
    from oracle import mxfp8 as o8
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.weights import interleave_row_groups, pack_mxfp8

    gc, gs = synthetic.mxfp8_tensor(seed, I, H, lead=(E,))
    uc, us = synthetic.mxfp8_tensor(seed + 1, I, H, lead=(E,))
    dc, ds = synthetic.mxfp8_tensor(seed + 2, H, I, lead=(E,))
    gu_q, gu_s = pack_mxfp8(interleave_row_groups(gc, uc), interleave_row_groups(gs, us))
    dn_q, dn_s = pack_mxfp8(dc, ds)
    gate, up = o8.dequantize_mxfp8_to_bf16(gc, gs), o8.dequantize_mxfp8_to_bf16(uc, us)
    gu_ref = torch.stack([gate.transpose(1, 2), up.transpose(1, 2)], 2).contiguous()
    dn_ref = o8.dequantize_mxfp8_to_bf16(dc, ds).transpose(1, 2).contiguous()
    gb = (synthetic.normal_bf16(seed + 3, (E, 2, I)).float() * 0.05).to(torch.bfloat16)
    db = (synthetic.normal_bf16(seed + 4, (E, H)).float() * 0.05).to(torch.bfloat16)
    return (gu_q, gu_s, dn_q, dn_s, gb, db), (gu_ref, dn_ref, gb, db.unsqueeze(1))


@pytest.mark.parametrize("E,k,H,I,T,block", [(8, 2, 256, 512, 300, 256), (6, 2, 416, 288, 77, 128)])
def test_moe_cte_mxfp8_weights(dev, E, k, H, I, T, block):
    """moe_cte with MXFP8 expert weights (the MxFP8 format of the reference's
    shard_on_block_mx kernel, moe_cte.py:136-138) against the oracle's dense torch flow
    (moe_cte.py:448-581) on the weights the MX definition dequantizes to; partial K chunks
    and N-tiles in the second case."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic

    from oracle import blockwise as ob
    from oracle import moe_cte as oc

    (gu_q, gu_s, dn_q, dn_s, gb, db), (gu_ref, dn_ref, gb_ref, db_ref) = _mxfp8_experts(
        71 + H, E, H, I)
    x = synthetic.tokens(71, T, H)
    logits = synthetic.normal_bf16(72, (T, E)).float()
    top = torch.topk(logits, k, dim=1)
    aff = torch.zeros(T, E).scatter_(1, top.indices, torch.softmax(top.values, 1))
    am_g, tp, b2e, cond = NF.build_blockwise_mapping(aff.to(dev), E, k, block)
    mv = lambda t: t.to(dev)  # noqa: E731
    got = NF.moe_cte(x.to(dev), am_g, mv(gu_q), mv(dn_q), tp, b2e, block, conditions=cond,
                     gate_and_up_proj_bias=mv(gb), down_proj_bias=mv(db),
                     gate_up_proj_scale=mv(gu_s), down_proj_scale=mv(dn_s),
                     activation_function="Swish", skip_token=True,
                     expert_affinities_scaling_mode="POST_SCALE", gate_clamp_upper_limit=7.0,
                     up_clamp_upper_limit=8.0, up_clamp_lower_limit=-6.0).cpu()
    am_r, _, _, _ = ob.build_blockwise_mapping(aff, E, k, block)
    want = oc.torch_moe_impl(x, am_r, gu_ref, dn_ref, gb_ref, db_ref,
                             gate_clamp_upper_limit=7.0, up_clamp_upper_limit=8.0,
                             up_clamp_lower_limit=-6.0, activation_function="Swish")
    check_close(got, want, None, f"moe_cte MXFP8 E={E} H={H} I={I}")


def test_decode_rejects_mxfp8_weights(dev):
    """The decode operators take MXFP4 experts only, as the reference's decode kernel does
    (moe_tkg.py:48)."""
    from vllm_neuron_amd import functional as NF

    (gu_q, gu_s, dn_q, dn_s, gb, db), _ = _mxfp8_experts(5, 4, 256, 256)
    x = torch.zeros(4, 256, dtype=torch.bfloat16, device=dev)
    aff = torch.zeros(4, 4, device=dev)
    idx = torch.zeros(4, 2, dtype=torch.int32, device=dev)
    mv = lambda t: t.to(dev)  # noqa: E731
    with pytest.raises(NotImplementedError, match="MXFP8"):
        NF.moe_tkg(x, mv(gu_q), mv(dn_q), aff, idx, is_all_expert=False,
                   expert_gate_up_weights_scale=mv(gu_s), expert_down_weights_scale=mv(dn_s))
