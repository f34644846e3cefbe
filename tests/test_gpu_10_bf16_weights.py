"""bf16 expert weights (the reference's shard_on_block operands; the bf16 GPT-OSS model's
prefill call model_bf16.py:1360-1391 and decode call :1199-1252) through moe_cte and
moe_block_tkg, and the dense mlp with quantization NONE, against the oracle's torch flows
on the same bf16 weights (moe_cte.py:448-581; moe_block_tkg.py:56-302; mlp.py:371-418).  Bounds: normalized max 2e-2, mean 5e-3
(tests/moe_helpers.check_close)."""

import pytest
import torch

from moe_helpers import check_close

pytestmark = pytest.mark.gpu


def _bf16_experts(seed, E, H, I, bias_scale=0.05):
    """gate_up [E, H, 2I] (gate columns, then up), down [E, I, H], biases [E, 2I] and
    [E, H]: the bf16 model's parameter shapes (model_bf16.py:1086-1115)."""
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, std: (torch.randn(*s, generator=g) * std).to(torch.bfloat16)  # noqa: E731
    return (r(E, H, 2 * I, std=H ** -0.5), r(E, I, H, std=I ** -0.5),
            r(E, 2 * I, std=bias_scale), r(E, H, std=bias_scale))


def _route(seed, T, E, k):
    from vllm_neuron_amd import synthetic

    logits = synthetic.normal_bf16(seed, (T, E)).float()
    top = torch.topk(logits, k, dim=1)
    return torch.zeros(T, E).scatter_(1, top.indices, torch.softmax(top.values, 1))


CASES = [
    # E, k, H, I, T, block, activation, clamps, biases
    (8, 2, 256, 512, 300, 256, "Swish", True, True),
    (6, 2, 416, 288, 77, 128, "SiLU", False, True),    # K and N tails in both GEMMs
    (4, 1, 96, 64, 129, 512, "GELU", False, False),
    (3, 3, 128, 96, 1, 128, "Swish", True, True),      # one token
    (2, 1, 32, 32, 5, 128, "SiLU", False, True),       # smallest K and N: one partial chunk
]


@pytest.mark.parametrize("E,k,H,I,T,block,act,clamp,biases", CASES)
def test_moe_cte_bf16_weights(dev, E, k, H, I, T, block, act, clamp, biases):
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.enums import MoECTEImplementation

    from oracle import blockwise as ob
    from oracle import moe_cte as oc

    print(f"moe_cte bf16 E={E} k={k} H={H} I={I} T={T} block={block} {act}", flush=True)
    gu, dn, gb, db = _bf16_experts(80 + H + I, E, H, I)
    x = synthetic.tokens(81, T, H)
    aff = _route(82 + T, T, E, k)
    lim = dict(gate_clamp_upper_limit=7.0, up_clamp_upper_limit=8.0,
               up_clamp_lower_limit=-6.0) if clamp else {}
    am_g, tp, b2e, cond = NF.build_blockwise_mapping(aff.to(dev), E, k, block)
    mv = lambda t: t.to(dev)  # noqa: E731
    got = NF.moe_cte(implementation=MoECTEImplementation.shard_on_block, conditions=cond,
                     hidden_states=x.to(dev), expert_affinities_masked=am_g,
                     gate_up_proj_weight=mv(gu).reshape(E, H, 2, I), down_proj_weight=mv(dn),
                     gate_and_up_proj_bias=mv(gb).reshape(E, 2, I) if biases else None,
                     down_proj_bias=mv(db).unsqueeze(1) if biases else None,
                     activation_function=act, block_size=block, token_position_to_id=tp,
                     block_to_expert=b2e, expert_affinities_scaling_mode="POST_SCALE",
                     skip_token=True, is_tensor_update_accumulating=True, **lim).cpu()
    am_r, _, _, _ = ob.build_blockwise_mapping(aff, E, k, block)
    want = oc.torch_moe_impl(x, am_r, gu.reshape(E, H, 2, I), dn,
                             gb.reshape(E, 2, I) if biases else None,
                             db.unsqueeze(1) if biases else None, activation_function=act, **lim)
    assert got.dtype == torch.bfloat16
    check_close(got.float(), want.float(), None, f"moe_cte bf16 E={E} H={H} I={I} T={T}")


def test_moe_cte_bf16_weights_gptoss20b_shape(dev):
    """20B-shaped layer (E=32, top-4, H = I = 2880, clamped Swish) at 2,048 tokens: the
    partial last K chunk (2880 = 22.5 x 128) and down N-tile; sampled rows through the
    routed form of the same flow."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic

    from oracle import blockwise as ob
    from oracle import moe_cte as oc

    E, k, H, I, T = 32, 4, 2880, 2880, 2048
    gu, dn, gb, db = _bf16_experts(90, E, H, I)
    x = synthetic.tokens(91, T, H)
    aff = _route(92, T, E, k)
    lim = dict(gate_clamp_upper_limit=7.0, up_clamp_upper_limit=8.0, up_clamp_lower_limit=-6.0)
    am_g, tp, b2e, cond = NF.build_blockwise_mapping(aff.to(dev), E, k, 256)
    got = NF.moe_cte(x.to(dev), am_g, gu.to(dev).reshape(E, H, 2, I), dn.to(dev), tp, b2e, 256,
                     implementation="shard_on_block", gate_and_up_proj_bias=gb.to(dev),
                     down_proj_bias=db.to(dev), activation_function="Swish", **lim).cpu()
    rows = torch.arange(0, T, 37)
    am_r, _, _, _ = ob.build_blockwise_mapping(aff, E, k, 256)
    want = oc.torch_moe_impl_routed(x, am_r, gu.reshape(E, H, 2, I), dn, gb.reshape(E, 2, I),
                                    db.unsqueeze(1), activation_function="Swish",
                                    token_rows=rows, **lim)
    check_close(got[rows].float(), want, None, "moe_cte bf16 20b shape")


@pytest.mark.parametrize("mode", ["PRE_SCALE", "PRE_SCALE_DELAYED"])
def test_moe_cte_bf16_weights_prescale_modes(dev, mode):
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic

    from oracle import blockwise as ob
    from oracle import moe_cte as oc

    E, k, H, I, T = 8, 2, 256, 384, 200
    gu, dn, gb, db = _bf16_experts(95, E, H, I, bias_scale=1.0)
    x = synthetic.tokens(96, T, H)
    aff16 = _route(97, T, E, k).to(torch.bfloat16)
    am_g, tp, b2e, cond = NF.build_blockwise_mapping(aff16.float().to(dev), E, k, 256)
    got = NF.moe_cte(x.to(dev), am_g, gu.to(dev).reshape(E, H, 2, I), dn.to(dev), tp, b2e, 256,
                     implementation="shard_on_block", gate_and_up_proj_bias=gb.to(dev),
                     down_proj_bias=db.to(dev), activation_function="Swish",
                     expert_affinities_scaling_mode=mode, gate_clamp_upper_limit=7.0).cpu()
    am_r, _, _, _ = ob.build_blockwise_mapping(aff16.float(), E, k, 256)
    want = oc.torch_moe_impl(x, am_r.to(torch.bfloat16), gu.reshape(E, H, 2, I), dn,
                             gb.reshape(E, 2, I), db.unsqueeze(1), gate_clamp_upper_limit=7.0,
                             activation_function="Swish", expert_affinities_scaling_mode=mode)
    check_close(got.float(), want.float(), None, f"moe_cte bf16 {mode}")


def test_bf16_model_prefill_call_chain(dev):
    """The bf16 GPT-OSS model's prefill MoE (model_bf16.py:1282-1391) with its argument
    lists: router (fp32 softmax routing) -> build_blockwise_mapping -> moe_cte
    (shard_on_block, reshaped [E, H, 2I] parameters, [E, 2I] / [E, H] biases) against the
    oracle's router, mapping and moe_cte torch flows."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.enums import ExpertAffinityScaleMode, MoECTEImplementation

    from oracle import blockwise as ob
    from oracle import moe_cte as oc
    from oracle import router as orr

    E, k, H, I, T, block, limit = 16, 4, 512, 384, 333, 256, 7.0
    gu, dn, gb, db = _bf16_experts(98, E, H, I)
    x = synthetic.tokens(99, T, H)
    rw = synthetic.normal_bf16(100, (E, H), 0.02)
    rb = synthetic.normal_bf16(101, (E,), 0.02)
    mv = lambda t: t.to(dev)  # noqa: E731
    aff = NF.router(hidden_states=x.to(dev), router_weights=mv(rw).T, top_k=k,
                    router_bias=mv(rb), activation="softmax", computation_dtype=torch.float32)
    am, tp, b2e, cond = NF.build_blockwise_mapping(expert_affinities=aff, num_local_experts=E,
                                                   num_experts_per_token=k, block_size=block)
    got = NF.moe_cte(
        implementation=MoECTEImplementation.shard_on_block, conditions=cond,
        hidden_states=x.to(dev), expert_affinities_masked=am,
        gate_up_proj_weight=mv(gu).reshape(E, H, 2, I), down_proj_weight=mv(dn),
        gate_and_up_proj_bias=mv(gb).reshape(E, 2, I), down_proj_bias=mv(db).unsqueeze(1),
        activation_function="Swish", block_size=block,
        token_position_to_id=tp.to(dtype=torch.int32), block_to_expert=b2e.to(dtype=torch.int32),
        expert_affinities_scaling_mode=ExpertAffinityScaleMode.POST_SCALE, skip_token=True,
        gate_clamp_upper_limit=limit, gate_clamp_lower_limit=None,
        up_clamp_upper_limit=limit + 1, up_clamp_lower_limit=-limit + 1,
        is_tensor_update_accumulating=True, compute_dtype="bfloat16").cpu()
    aff_r = orr.router(x, rw.T, k, rb, "softmax", computation_dtype=torch.float32)
    assert torch.equal(aff.cpu() != 0, aff_r != 0), "selected experts differ"
    am_r, _, _, _ = ob.build_blockwise_mapping(aff_r, E, k, block)
    want = oc.torch_moe_impl(x, am_r, gu.reshape(E, H, 2, I), dn, gb.reshape(E, 2, I),
                             db.unsqueeze(1), gate_clamp_upper_limit=limit,
                             up_clamp_upper_limit=limit + 1, up_clamp_lower_limit=-limit + 1,
                             activation_function="Swish")
    check_close(got.float(), want.float(), None, "bf16 model prefill chain")


@pytest.mark.parametrize("T,H,I,act,bias", [(1, 256, 384, "SiLU", True), (200, 416, 288, "GELU", False),
                                            (1000, 2880, 2880, "SiLU", True)])
def test_mlp_bf16_weights(dev, T, H, I, act, bias):
    """Dense mlp with quantization NONE (bf16 gate_w / up_w [H, I], down_w [I, H]) against
    the reference's torch flow (mlp.py:371-418)."""
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.enums import QuantizationType
    from vllm_neuron_amd.functional import mlp

    from oracle import mlp as om

    print(f"mlp bf16 T={T} H={H} I={I} {act}", flush=True)
    g = torch.Generator().manual_seed(110 + T)
    r = lambda *s, std: (torch.randn(*s, generator=g) * std).to(torch.bfloat16)  # noqa: E731
    gw, uw, dw = r(H, I, std=H ** -0.5), r(H, I, std=H ** -0.5), r(I, H, std=I ** -0.5)
    gb, ub, db = (r(1, I, std=0.1), r(1, I, std=0.1), r(1, H, std=0.1)) if bias else (None,) * 3
    x = synthetic.tokens(111, T, H)
    mv = lambda t: None if t is None else t.to(dev)  # noqa: E731
    got = mlp(x.to(dev), mv(gw), mv(uw), mv(dw), act_fn=act, gate_b=mv(gb), up_b=mv(ub),
              down_b=mv(db), quantization_type=QuantizationType.NONE).cpu()
    want = om.torch_mlp_impl(x, gw, uw, dw, act, gb, ub, db)
    assert got.dtype == torch.bfloat16 and got.shape == (T, H)
    check_close(got.float(), want.float(), None, f"mlp bf16 T={T} H={H} I={I}")


def test_moe_tkg_rejects_bf16_weights(dev):
    """moe_tkg takes MXFP4 experts only and raises for any other weights, as the reference
    does (moe_tkg.py:48, :191-194); moe_block_tkg takes bf16 experts (below)."""
    from vllm_neuron_amd import functional as NF

    gu, dn, _, _ = _bf16_experts(5, 4, 256, 256)
    x = torch.zeros(4, 256, dtype=torch.bfloat16, device=dev)
    aff = torch.zeros(4, 4, device=dev)
    idx = torch.zeros(4, 2, dtype=torch.int32, device=dev)
    with pytest.raises(NotImplementedError, match="MXFP4"):
        NF.moe_tkg(x, gu.to(dev).reshape(4, 256, 2, 256), dn.to(dev), aff, idx,
                   is_all_expert=False)


@pytest.mark.parametrize("T,E,k,H,I,act,pre_norm,scale", [
    (1, 16, 4, 512, 384, "SOFTMAX", False, "POST_SCALE"),
    (7, 8, 2, 416, 288, "SIGMOID", True, "NO_SCALE"),       # K and N tails in both GEMMs
    (64, 16, 4, 512, 384, "SOFTMAX", False, "POST_SCALE"),
    (3, 4, 2, 32, 32, "SOFTMAX", False, "POST_SCALE"),       # smallest K and N
])
def test_moe_block_tkg_bf16_weights(dev, T, E, k, H, I, act, pre_norm, scale):
    """moe_block_tkg with bf16 experts against the oracle's dense torch flow
    (moe_block_tkg.py:56-302: fp32 expert math over every expert, the output cast to
    bf16)."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic

    from oracle import moe_block_tkg as obt

    print(f"moe_block_tkg bf16 T={T} E={E} k={k} H={H} I={I} {act} {scale}", flush=True)
    gu, dn, gb, db = _bf16_experts(120 + T, E, H, I)
    x = synthetic.tokens(121 + T, T, H)
    gamma = 1.0 + 0.1 * torch.randn(H, generator=torch.Generator().manual_seed(122))
    rw = synthetic.normal_bf16(123, (H, E), 0.05)
    clamps = dict(gate_clamp_upper_limit=7.0, up_clamp_upper_limit=8.0,
                  up_clamp_lower_limit=-6.0)
    mv = lambda t: t.to(dev)  # noqa: E731
    out, logits = NF.moe_block_tkg(
        x.unsqueeze(0).to(dev), mv(gamma).unsqueeze(0), mv(rw), mv(gu).reshape(E, H, 2, I),
        mv(dn), top_k=k, expert_gate_up_bias=mv(gb).reshape(E, 2, I), expert_down_bias=mv(db),
        router_act_fn=act, router_pre_norm=pre_norm, expert_affinities_scaling_mode=scale,
        hidden_act_fn="Swish", **clamps)
    want, logits_r = obt.torch_moe_block_tkg_impl(
        x, gamma, rw, gu.reshape(E, H, 2, I), dn, expert_gate_up_bias=gb.reshape(E, 2, I),
        expert_down_bias=db, top_k=k, router_act_fn=act, router_pre_norm=pre_norm,
        expert_affinities_scaling_mode=scale, hidden_act_fn="Swish", **clamps)
    assert out.dtype == torch.bfloat16 and out.shape == (T, H)
    assert torch.allclose(logits.cpu(), logits_r, rtol=1e-5, atol=1e-5)
    check_close(out.cpu().float(), want.float(), None, f"moe_block_tkg bf16 T={T} {scale}")


def test_bf16_model_decode_call(dev):
    """The bf16 GPT-OSS model's decode MoE (model_bf16.py:1199-1252) with its argument list:
    padded H = I = 3072 with hidden_actual = 2880, fp32 gamma [1, H], router_weight.T, the
    bias views, softmax routing after top-k, clamped Swish; against the oracle's RMSNorm +
    router and its fp32 expert flow on the selected experts."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.enums import ActFnType, ExpertAffinityScaleMode, RouterActFnType

    from oracle import moe_block_tkg as obt

    E, k, H, I, ha, T, limit = 8, 4, 3072, 3072, 2880, 16, 7.0
    gu, dn, gb, db = _bf16_experts(130, E, H, I)
    x = synthetic.tokens(131, T, H)
    x[:, ha:] = 0
    ln_w = (1.0 + 0.1 * torch.randn(H, generator=torch.Generator().manual_seed(132))).to(
        torch.bfloat16)
    router_weight = synthetic.normal_bf16(133, (E, H), 0.05)
    router_bias = synthetic.normal_bf16(134, (E,), 0.05)
    mv = lambda t: t.to(dev)  # noqa: E731
    out = NF.moe_block_tkg(
        inp=x.to(dev).unsqueeze(0), gamma=mv(ln_w).unsqueeze(0).to(torch.float32),
        router_weights=mv(router_weight).T, expert_gate_up_weights=mv(gu).reshape(E, H, 2, I),
        expert_down_weights=mv(dn), rank_id=None, top_k=k,
        router_bias=mv(router_bias).unsqueeze(0),
        expert_gate_up_bias=mv(gb).reshape(E, 2, I), expert_down_bias=mv(db), eps=1e-5,
        router_act_fn=RouterActFnType.SOFTMAX, router_pre_norm=False,
        expert_affinities_scaling_mode=ExpertAffinityScaleMode.POST_SCALE,
        hidden_act_fn=ActFnType.Swish, gate_clamp_upper_limit=limit,
        gate_clamp_lower_limit=None, up_clamp_upper_limit=limit + 1,
        up_clamp_lower_limit=-limit + 1, router_mm_dtype="bfloat16", hidden_actual=ha,
        is_all_expert=False, skip_router_logits=True)
    xn, _, top, idx = obt.rmsnorm_router(x, ln_w.float(), router_weight.T, router_bias, 1e-5, k,
                                         "SOFTMAX", False, False, hidden_actual=ha)
    aff = torch.zeros(T, E).scatter_(1, idx, top)
    want = obt.expert_mlp_fp32_routed(xn, aff, gu.reshape(E, H, 2, I), dn, gb.reshape(E, 2, I),
                                      db, hidden_act_fn="Swish", gate_clamp_upper_limit=limit,
                                      up_clamp_upper_limit=limit + 1,
                                      up_clamp_lower_limit=-limit + 1, scale_mode="POST_SCALE",
                                      out_dtype=torch.bfloat16)
    got = out.cpu()
    assert got.shape == (T, H)
    check_close(got.float(), want.float(), None, "bf16 model decode call")


def _device_experts(dev, seed, E, H, I):
    """bf16 experts drawn on the GPU one expert at a time (gate_up [E, H, 2, I], down [E, I, H],
    biases [E, 2, I] / [E, H]): the 120B-shaped set is 6.4 GB."""
    g = torch.Generator(device=dev).manual_seed(seed)
    gu = torch.empty(E, H, 2, I, dtype=torch.bfloat16, device=dev)
    dn = torch.empty(E, I, H, dtype=torch.bfloat16, device=dev)
    for e in range(E):
        gu[e] = (torch.randn(H, 2, I, device=dev, generator=g) * H ** -0.5).to(torch.bfloat16)
        dn[e] = (torch.randn(I, H, device=dev, generator=g) * I ** -0.5).to(torch.bfloat16)
    gb = (torch.randn(E, 2, I, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    db = (torch.randn(E, H, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    return gu, dn, gb, db


def _subset(aff_rows, *tensors):
    """The experts the sampled rows select, ascending (the order the flows sum them in):
    affinities [rows, E_sub] and each [E, ...] tensor restricted to them, on the CPU."""
    sel = torch.nonzero((aff_rows != 0).any(0)).flatten()
    return (aff_rows[:, sel],) + tuple(t[sel.to(t.device)].cpu() for t in tensors)


def test_bf16_weights_gptoss120b_shape(dev):
    """120B-shaped layer with bf16 experts (E=128, top-4, H = I = 2880, clamped Swish):
    decode of 64 tokens through moe_block_tkg and prefill of 2,048 tokens through moe_cte,
    sampled rows against the oracle's flows over the experts those rows select."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic

    from oracle import blockwise as ob
    from oracle import moe_block_tkg as obt
    from oracle import moe_cte as oc

    E, k, H, I = 128, 4, 2880, 2880
    lim = dict(gate_clamp_upper_limit=7.0, up_clamp_upper_limit=8.0, up_clamp_lower_limit=-6.0)
    gu, dn, gb, db = _device_experts(dev, 140, E, H, I)
    rw = synthetic.normal_bf16(141, (H, E), 0.05)

    # decode
    T = 64
    x = synthetic.tokens(142, T, H)
    gamma = torch.ones(H)
    out = NF.moe_block_tkg(x.unsqueeze(0).to(dev), gamma.unsqueeze(0).to(dev), rw.to(dev), gu,
                           dn, top_k=k, expert_gate_up_bias=gb, expert_down_bias=db,
                           router_act_fn="SOFTMAX", router_pre_norm=False,
                           expert_affinities_scaling_mode="POST_SCALE", hidden_act_fn="Swish",
                           skip_router_logits=True, **lim).cpu()
    rows = torch.arange(0, T, 9)
    xn, _, top, idx = obt.rmsnorm_router(x, gamma, rw, None, 1e-6, k, "SOFTMAX", False, False)
    aff = torch.zeros(T, E).scatter_(1, idx, top)[rows]
    a_sub, gu_s, dn_s, gb_s, db_s = _subset(aff, gu, dn, gb, db)
    want = obt.expert_mlp_fp32_routed(xn[rows], a_sub, gu_s, dn_s, gb_s, db_s,
                                      hidden_act_fn="Swish", scale_mode="POST_SCALE",
                                      out_dtype=torch.bfloat16, **lim)
    check_close(out[rows].float(), want.float(), None, "bf16 experts 120b decode")

    # prefill
    T = 2048
    x = synthetic.tokens(143, T, H)
    aff = _route(144, T, E, k)
    am_g, tp, b2e, _ = NF.build_blockwise_mapping(aff.to(dev), E, k, 256)
    got = NF.moe_cte(x.to(dev), am_g, gu, dn, tp, b2e, 256, implementation="shard_on_block",
                     gate_and_up_proj_bias=gb, down_proj_bias=db, activation_function="Swish",
                     **lim).cpu()
    rows = torch.arange(0, T, 101)
    a_sub, gu_s, dn_s, gb_s, db_s = _subset(aff[rows], gu, dn, gb, db)
    want = oc.torch_moe_impl_routed(x[rows], a_sub.reshape(-1, 1), gu_s, dn_s, gb_s,
                                    db_s.unsqueeze(1), activation_function="Swish", **lim)
    check_close(got[rows].float(), want, None, "bf16 experts 120b prefill")


def test_moe_block_tkg_bf16_weights_graph_replays(dev):
    """The bf16-expert decode block (RMSNorm, router, scatter, mapping, both GEMMs, combine)
    captured in a HIP graph after one eager call: every replay, with eager work and
    synchronizations between them, equals the eager result for its input."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic

    E, k, H, I, T = 16, 4, 512, 384, 32
    gu, dn, gb, db = (t.to(dev) for t in _bf16_experts(150, E, H, I))
    rw = synthetic.normal_bf16(151, (H, E), 0.05).to(dev)
    gamma = torch.ones(1, H, device=dev)
    run = lambda x: NF.moe_block_tkg(  # noqa: E731
        x.unsqueeze(0), gamma, rw, gu.reshape(E, H, 2, I), dn, top_k=k,
        expert_gate_up_bias=gb.reshape(E, 2, I), expert_down_bias=db, router_act_fn="SOFTMAX",
        router_pre_norm=False, expert_affinities_scaling_mode="POST_SCALE",
        hidden_act_fn="Swish", skip_router_logits=True, gate_clamp_upper_limit=7.0)
    xs = [synthetic.tokens(152 + i, T, H).to(dev) for i in range(3)]
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
