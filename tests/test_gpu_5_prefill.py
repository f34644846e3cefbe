"""Prefill expert path (router -> blockwise mapping -> moe_cte) vs the oracle's
moe_cte torch flow (bf16 intermediates)."""

import pytest
import torch

from moe_helpers import build, check_close, routing_agreement

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
    got = layer.prefill(x.to(dev)).cpu()
    rows = torch.arange(0, T, max(1, T // 48))
    want = ref.prefill_routed(x, aff, token_rows=rows)
    check_close(got[rows], want, ties[rows], f"prefill 20b T={T} zipf={zipf}")


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
