"""The reference's own MXFP4 callers, run unchanged against this package's operators.

* GptOssExperts._run_moe_block_tkg (model_mxfp4.py:1158-1214) and the prefill chain of
  forward_prefill (:1333-1436), with their argument lists as written: tensors in the
  reference's Trainium MX parameter layout (:957-1018, padded H = I = 3072 with
  hidden_actual = 2880), fp16 router weight and bias (:950-955), the tiled gate/up bias
  view, router(computation_dtype=float16), build_blockwise_mapping with moe_group and
  tp_degree, conditions padded by two.
* The fp16 / bf16 router computations, router(gamma=...), rmsnorm_router_topk_tkg, and
  the decode front end's selected experts with fp16 router weights.

Every result is compared with the oracle on the true (unpadded) layer: routing indices
exactly (near-ties of the oracle's scores exempted and counted), layer outputs within
max 2e-2 / mean 5e-3 normalized, padded output columns exactly zero.
"""

import math

import pytest
import torch

from moe_helpers import aff_close, check_close, check_indices, near_tie
from oracle import blockwise as obw
from oracle import moe_block_tkg as obt
from oracle import neuron_layout as onl
from oracle import rmsnorm_router_topk as ort
from oracle import router as orr
from oracle.layer import RefLayer

pytestmark = pytest.mark.gpu

H_PAD = I_PAD = 3072  # GPT-OSS padding of the reference's Trainium model (config.py:115-119)


class NeuronParams:
    """The parameters GptOssExperts (model_mxfp4.py:947-1018) holds after loading one layer
    of a GPT-OSS checkpoint, built with the oracle's restatement of the loaders."""

    def __init__(self, lt, dev, seed):
        from vllm_neuron_amd import synthetic

        E = lt.gate_up_blocks.shape[0]
        self.E = E
        self.gate_up_proj_weight = onl.gate_up_blocks(lt.gate_up_blocks, H_PAD, I_PAD).to(dev)
        self.gate_up_proj_scale = onl.gate_up_scales(lt.gate_up_scales, H_PAD, I_PAD).to(dev)
        self.gate_up_proj_bias = onl.gate_up_bias(lt.gate_up_bias, I_PAD).to(dev)
        self.down_proj_weight = onl.down_blocks(lt.down_blocks, H_PAD, I_PAD).to(dev)
        self.down_proj_scale = onl.down_scales(lt.down_scales, H_PAD, I_PAD).to(dev)
        self.down_proj_bias = onl.down_bias(lt.down_bias, H_PAD).to(dev)
        H = lt.router_w.shape[1]
        self.router_w16 = lt.router_w.to(torch.float16)  # [E, H], the model's fp16 parameter
        rw = torch.zeros(E, H_PAD, dtype=torch.float16)
        rw[:, :H] = self.router_w16
        self.router_weight = rw.to(dev)
        self.router_b16 = synthetic.normal_bf16(seed, (E,), 0.5).to(torch.float16)
        self.router_bias = self.router_b16.to(dev)
        g = 1.0 + 0.1 * torch.randn(H, generator=torch.Generator().manual_seed(seed))
        self.gamma = g.to(torch.bfloat16)  # GptOssRMSNorm weight (model dtype)
        gp = torch.zeros(H_PAD, dtype=torch.bfloat16)
        gp[:H] = self.gamma
        self.ln_weight = gp.to(dev)


@pytest.fixture(scope="module")
def layer20(dev):
    from vllm_neuron_amd import synthetic

    lt = synthetic.layer_tensors(synthetic.GPT_OSS_20B, 61)
    return lt, RefLayer(lt), NeuronParams(lt, dev, 62)


def _norm_stage(xn_g, x, gamma, eps, ha, all_cols):
    """The GPU's RMSNorm rows against the oracle's: within one bf16 rounding step, almost
    all bit-identical.  Later stages are then checked from the GPU's own rows."""
    if all_cols:
        xn_r = orr.rms_norm(x, gamma, eps)
    else:
        xn_r, _, _, _ = obt.rmsnorm_router(x, gamma, torch.zeros(x.shape[1], 1), None, eps, 1,
                                           "SOFTMAX", False, False, hidden_actual=ha)
    d = (xn_g.float() - xn_r.float()).abs()
    ulp = torch.ldexp(torch.ones_like(d), torch.frexp(xn_r.float()).exponent - 8)
    assert bool((d <= ulp).all())
    same = (d == 0).float().mean().item()
    print(f"RMSNorm rows bit-identical: {same:.5f}")
    assert same > 0.99
    return xn_r


def _pad_cols(x):
    out = torch.zeros(x.shape[0], H_PAD, dtype=x.dtype)
    out[:, :x.shape[1]] = x
    return out


def _block_tkg_kwargs(p, hidden_states, H, dev):
    """The keyword arguments of _run_moe_block_tkg's NF.moe_block_tkg call
    (model_mxfp4.py:1183-1214) on the parameters p."""
    from vllm_neuron_amd.enums import ActFnType, ExpertAffinityScaleMode, RouterActFnType

    limit, K, E = 7.0, 4, p.E
    I_TP = p.gate_up_proj_weight.shape[-1]
    n_blk = math.ceil(I_TP / 512.0)
    blk = I_TP // n_blk
    rank_id = torch.tensor([[0]], dtype=torch.int32, device=dev)
    return dict(
        inp=hidden_states.unsqueeze(0),
        gamma=p.ln_weight.unsqueeze(0).to(torch.float32),
        router_weights=p.router_weight.T,
        expert_gate_up_weights=p.gate_up_proj_weight,
        expert_down_weights=p.down_proj_weight,
        rank_id=rank_id,
        top_k=K,
        expert_gate_up_weights_scale=p.gate_up_proj_scale,
        expert_down_weights_scale=p.down_proj_scale,
        router_bias=p.router_bias.unsqueeze(0),
        expert_gate_up_bias=p.gate_up_proj_bias.view(E, blk // 4, 2, n_blk, 4),
        expert_down_bias=p.down_proj_bias,
        eps=1e-5,
        router_act_fn=RouterActFnType.SOFTMAX,
        router_pre_norm=False,
        expert_affinities_scaling_mode=ExpertAffinityScaleMode.POST_SCALE,
        hidden_act_fn=ActFnType.Swish,
        gate_clamp_upper_limit=limit,
        gate_clamp_lower_limit=None,
        up_clamp_upper_limit=limit + 1,
        up_clamp_lower_limit=-limit + 1,
        router_mm_dtype=torch.float16,
        hidden_actual=H,
        is_all_expert=True,
        skip_router_logits=True,
    )


@pytest.mark.parametrize("T", [8, 64])
def test_model_mxfp4_decode_call(dev, layer20, T):
    """_run_moe_block_tkg's NF.moe_block_tkg call (model_mxfp4.py:1183-1214) verbatim."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic

    lt, ref, p = layer20
    H = ref.H
    K, E = 4, p.E
    x = synthetic.tokens(63, T, H)
    hidden_states = _pad_cols(x).to(dev)
    kw = _block_tkg_kwargs(p, hidden_states, H, dev)
    out = NF.moe_block_tkg(**kw)
    assert out.shape == (T, H_PAD) and out.dtype == torch.bfloat16
    kw["skip_router_logits"] = False
    out2, logits = NF.moe_block_tkg(**kw)  # converted weights now come from the cache
    assert torch.equal(out, out2)
    out = out.cpu()
    assert torch.all(out[:, H:] == 0)
    # the block's RMSNorm stage (same kernel as NF.rmsnorm) against the oracle's
    xn_g = NF.rmsnorm(hidden_states, kw["gamma"], 1e-5, hidden_actual=H).cpu()
    assert torch.all(xn_g[:, H:] == 0)
    _norm_stage(xn_g[:, :H], x, p.gamma.float(), 1e-5, H, all_cols=False)
    # the router stage on those rows: the oracle's fp32 flow (moe_block_tkg.py:152-204)
    logits_r = xn_g[:, :H].float() @ p.router_w16.T.float() + p.router_b16.float()
    top, idx = torch.topk(logits_r, K, dim=1)
    top = torch.softmax(top, dim=1)
    assert torch.allclose(logits.cpu(), logits_r, rtol=1e-5, atol=1e-5)
    aff = torch.zeros(T, E).scatter_(1, idx, top)
    want = ref.decode_routed(xn_g[:, :H], aff)
    ties = torch.tensor([near_tie(logits_r[t], K) for t in range(T)])
    check_close(out[:, :H], want, ties, f"model_mxfp4 decode call T={T}")


def test_model_mxfp4_in_place_experts(dev, layer20):
    """With in-place conversion on, the model's Trainium-layout parameters are rewritten
    into packed bytes in their own memory on the first call (no converted copy is kept),
    and the decode call gives the copy path's output bit for bit, on the first call and
    on later ones."""
    import types

    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.functional.moe import _cache
    from vllm_neuron_amd.neuron_layout import packed_in_place, set_convert_in_place

    lt, ref, p = layer20
    H = ref.H
    x = synthetic.tokens(64, 16, H)
    hidden_states = _pad_cols(x).to(dev)
    want = NF.moe_block_tkg(**_block_tkg_kwargs(p, hidden_states, H, dev))
    q = types.SimpleNamespace(**vars(p))
    for n in ("gate_up_proj_weight", "gate_up_proj_scale", "down_proj_weight",
              "down_proj_scale"):
        setattr(q, n, getattr(p, n).clone())
    ptr = q.gate_up_proj_weight.data_ptr()
    prev = set_convert_in_place(True)
    try:
        n0 = _cache.entries()
        got = NF.moe_block_tkg(**_block_tkg_kwargs(q, hidden_states, H, dev))
        assert packed_in_place(q.gate_up_proj_weight, q.gate_up_proj_scale,
                               q.down_proj_weight, q.down_proj_scale) is not None
        assert q.gate_up_proj_weight.data_ptr() == ptr
        assert torch.equal(got, want)
        got2 = NF.moe_block_tkg(**_block_tkg_kwargs(q, hidden_states, H, dev))
        assert torch.equal(got2, want)
        # only the two bias conversions were cached, no expert copy
        assert _cache.entries() <= n0 + 2
    finally:
        set_convert_in_place(prev)


def test_model_mxfp4_prefill_chain(dev, layer20):
    """forward_prefill's router -> build_blockwise_mapping -> moe_cte calls
    (model_mxfp4.py:1337-1436) verbatim, from the normalized hidden states on."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.enums import ActFnType, ExpertAffinityScaleMode, MoECTEImplementation

    lt, ref, p = layer20
    H, T, K, E, limit = ref.H, 700, 4, p.E, 7.0
    x = synthetic.tokens(64, T, H)
    hidden_states = _pad_cols(x).to(dev)
    positions = torch.cat([torch.arange(650), torch.zeros(50, dtype=torch.int64)]).to(dev)
    expert_affinities = NF.router(hidden_states=hidden_states, router_weights=p.router_weight.T,
                                  top_k=K, router_bias=p.router_bias, activation="softmax",
                                  computation_dtype=torch.float16)
    _, logits_g = NF.router(hidden_states, p.router_weight.T, K, p.router_bias, "softmax",
                            return_logits=True, computation_dtype=torch.float16)
    last_real_idx = torch.argmax(positions)
    padding_mask = torch.arange(positions.shape[0], device=dev) <= last_real_idx
    (expert_affinities_masked, token_position_to_id, block_to_expert,
     conditions) = NF.build_blockwise_mapping(expert_affinities=expert_affinities,
                                              num_local_experts=E, num_experts_per_token=K,
                                              block_size=256, moe_group=None, tp_degree=1,
                                              padding_mask=padding_mask)
    conditions = torch.cat([conditions, torch.zeros(2, device=conditions.device)])
    I_TP = p.gate_up_proj_weight.shape[-1]
    n_blk = math.ceil(I_TP / 512)
    blk = I_TP // n_blk
    output = NF.moe_cte(
        implementation=MoECTEImplementation.shard_on_block_mx, conditions=conditions,
        hidden_states=hidden_states, expert_affinities_masked=expert_affinities_masked,
        gate_up_proj_weight=p.gate_up_proj_weight, down_proj_weight=p.down_proj_weight,
        gate_and_up_proj_bias=p.gate_up_proj_bias.reshape(E, blk // 4, 2, n_blk, 4),
        down_proj_bias=p.down_proj_bias, activation_function=ActFnType.Swish, block_size=256,
        token_position_to_id=token_position_to_id.to(dtype=torch.int32),
        block_to_expert=block_to_expert.to(dtype=torch.int32),
        gate_up_proj_scale=p.gate_up_proj_scale, down_proj_scale=p.down_proj_scale,
        expert_affinities_scaling_mode=ExpertAffinityScaleMode.POST_SCALE, skip_token=True,
        gate_clamp_upper_limit=limit, gate_clamp_lower_limit=None,
        up_clamp_upper_limit=limit + 1, up_clamp_lower_limit=-limit + 1,
        is_tensor_update_accumulating=True, compute_dtype=torch.bfloat16).cpu()
    assert output.shape == (T, H_PAD)
    # router in fp16, as the oracle's torch flow computes it
    aff_r, logits_r = orr.router(x, p.router_w16.T, K, p.router_b16, "softmax",
                                 return_logits=True, computation_dtype=torch.float16)
    aff_g = expert_affinities.cpu()
    assert aff_g.dtype == torch.float16
    sel_g, sel_r = aff_g != 0, aff_r != 0
    bad = (sel_g != sel_r).any(1)
    for t in torch.nonzero(bad).flatten().tolist():
        srt = torch.sort(logits_r[t].float(), descending=True).values
        assert float(srt[K - 1] - srt[K]) <= 2 * 2.0 ** (math.floor(math.log2(abs(float(srt[K - 1])) + 1e-30)) - 10), t
    print(f"fp16 router: {int(bad.sum())} of {T} tokens select differently at a 1-ulp tie")
    ok = ~bad
    aff_close(aff_g[ok], aff_r[ok], logits_g.cpu()[ok], logits_r[ok], 2.0 ** -11)
    # layer output on the real tokens, from the oracle's routing
    aff_r[650:] = 0  # padding tokens route nowhere
    rows = torch.arange(0, T, 5)
    rows = rows[ok[rows]]
    want = ref.prefill_routed(x, aff_r.float(), token_rows=rows)
    assert torch.all(output[:, H:] == 0)
    assert torch.all(output[650:] == 0)
    real = rows[rows < 650]
    check_close(output[real, :H].float(), want[:len(real)], None, "model_mxfp4 prefill chain")


@pytest.mark.parametrize("cdt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("wdt", [torch.float16, torch.bfloat16])
def test_router_computation_dtypes(dev, cdt, wdt):
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic

    T, E, K, H = 512, 128, 4, 2880
    x = synthetic.normal_bf16(71, (T, H))
    w = synthetic.normal_bf16(72, (E, H), 0.02).to(wdt)
    b = synthetic.normal_bf16(73, (E,), 0.5).to(wdt)
    aff_g, logits_g = NF.router(x.to(dev), w.to(dev).T, K, b.to(dev), "softmax",
                                return_logits=True, computation_dtype=cdt)
    aff_r, logits_r = orr.router(x, w.T, K, b, "softmax", return_logits=True,
                                 computation_dtype=cdt)
    assert aff_g.dtype == cdt and logits_g.dtype == cdt
    lg, lr = logits_g.cpu().double(), logits_r.double()
    if cdt == torch.float32:
        assert torch.allclose(lg, lr, rtol=1e-5, atol=1e-5)
        tol = 1e-6
    else:
        mant = 10 if cdt == torch.float16 else 7
        ulp = torch.pow(2.0, torch.floor(torch.log2(lr.abs().clamp(min=1e-30))) - mant)
        if cdt == torch.float16:
            ulp = ulp.clamp(min=2.0 ** -24)  # fp16 subnormal spacing
        # one rounding step apart, plus the fp32 summation-order error of the two sums
        # (absolute: about 2^-24 of the sum of |products|, ~40 here), which dominates
        # near zero, where a logit is a small difference of large sums
        sum_abs = (x.float().abs() @ w.float().abs().T).double() + b.float().abs().double()
        slack = 8 * 2.0 ** -24 * sum_abs
        d = (lg - lr).abs()
        assert bool((d <= ulp + slack).all()), float((d - ulp - slack).max())
        same = (logits_g.cpu() == logits_r).double().mean().item()
        print(f"logits bit-identical: {same:.5f}")
        assert same > 0.99
        tol = 2.0 ** -(mant + 1)
    idx_r = torch.topk(logits_r.float(), K, dim=1).indices
    idx_g = torch.topk(logits_g.cpu().float(), K, dim=1).indices
    sel_g = torch.zeros(T, E, dtype=torch.bool).scatter_(1, idx_g, True)
    sel_r = torch.zeros(T, E, dtype=torch.bool).scatter_(1, idx_r, True)
    bad = (sel_g != sel_r).any(1) | ((aff_g.cpu() != 0) != (aff_r != 0)).any(1)
    for t in torch.nonzero(bad).flatten().tolist():
        srt = torch.sort(lr[t], descending=True).values
        assert float(srt[K - 1] - srt[K]) <= 2 * (tol * 2 * max(1.0, abs(float(srt[0])))), t
    print(f"cdt={cdt} w={wdt}: {int(bad.sum())} of {T} tokens at a tie")
    if cdt != torch.bfloat16:  # bf16 logits tie often; torch.topk then picks either
        assert int(bad.sum()) <= T // 50
    ok = ~bad
    aff_close(aff_g.cpu()[ok], aff_r[ok], logits_g.cpu()[ok], logits_r[ok], 2 * tol)


def test_router_gamma(dev):
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic

    T, E, K, H = 256, 32, 4, 2880
    x = synthetic.normal_bf16(74, (T, H))
    w = synthetic.normal_bf16(75, (E, H), 0.02)
    gamma = 1.0 + 0.1 * torch.randn(H, generator=torch.Generator().manual_seed(76))
    from vllm_neuron_amd.functional.moe.router import rms_norm

    aff_g, logits_g = NF.router(x.to(dev), w.to(dev).T, K, gamma=gamma.to(dev), eps=1e-5,
                                return_logits=True)
    # the RMSNorm stage router(gamma) runs first, against the oracle's (router.py:680-687)
    xn_g = rms_norm(x.to(dev), gamma.to(dev), 1e-5).cpu()
    _norm_stage(xn_g, x, gamma.float(), 1e-5, None, all_cols=True)
    # the router stage from those rows
    aff_r, logits_r = orr.router(xn_g, w.T, K, return_logits=True)
    assert torch.allclose(logits_g.cpu(), logits_r, rtol=1e-5, atol=1e-5)
    idx_g = torch.topk(aff_g.cpu(), K, dim=1).indices.sort(1).values
    idx_r = torch.topk(aff_r, K, dim=1).indices.sort(1).values
    bad = check_indices(idx_g, logits_r, idx_r, K, "router(gamma)")
    aff_close(aff_g.cpu()[~bad], aff_r[~bad], logits_g.cpu()[~bad], logits_r[~bad], 1e-6)


@pytest.mark.parametrize("mm", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("fn,ha,T", [("SOFTMAX", 2880, 64), ("SIGMOID", None, 16),
                                      ("SOFTMAX", 2800, 300)])
def test_rmsnorm_router_topk_tkg(dev, mm, fn, ha, T):
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.enums import RouterActFnType

    E, K, H = 128, 4, 3072
    x = synthetic.normal_bf16(77, (1, T, H))
    w = synthetic.normal_bf16(78, (E, H), 0.02).to(torch.float16)
    b = synthetic.normal_bf16(79, (1, E), 0.5).to(torch.float16)
    gamma = (1.0 + 0.1 * torch.randn(1, H, generator=torch.Generator().manual_seed(80))).float()
    norm_g, idx_g, aff_g = NF.rmsnorm_router_topk_tkg(
        x.to(dev), gamma.to(dev), w.to(dev).T, b.to(dev), eps=1e-5, top_k=K, hidden_actual=ha,
        router_mm_dtype=mm, router_act_fn=RouterActFnType[fn])
    norm_r, idx_r, aff_r, logits_r = ort.rmsnorm_router_topk(x, gamma, w.T, b, 1e-5, K, ha, mm,
                                                             fn)
    assert norm_g.dtype == mm and aff_g.dtype == torch.bfloat16 and idx_g.dtype == torch.int32
    ng, nr = norm_g.cpu().double(), norm_r.double()
    mant = 10 if mm == torch.float16 else 7
    ulp = torch.pow(2.0, torch.floor(torch.log2(nr.abs().clamp(min=1e-30))) - mant)
    assert bool(((ng - nr).abs() <= ulp).all())
    assert (norm_g.cpu() == norm_r).double().mean().item() > 0.99
    # the router stage from the GPU's own norm (fp64 products of the cast operands)
    lf = ng @ w.T.to(mm).double() + b.to(mm).double()
    vals, idx_f = torch.topk(lf, K, dim=1)
    bad = check_indices(idx_g, lf, idx_f, K, f"rmsnorm_router_topk mm={mm}")
    ok = ~bad
    if fn == "SOFTMAX":
        probs = torch.softmax(vals, dim=1)
    else:
        probs = torch.sigmoid(vals)
    exact = torch.zeros(T, E, dtype=torch.float64).scatter_(1, idx_f, probs)
    d = (aff_g.cpu()[ok].double() - exact[ok]).abs()
    assert float(d.max()) <= 2.0 ** -9  # half a bf16 ulp below 1


@pytest.mark.parametrize("T", [8, 64, 200])
def test_block_decode_selected_experts_fp16_router(dev, T):
    """The decode front end's selected experts (topk_idx_out of mxmoe_moe_block_decode)
    with the model's fp16 router weight and bias, through the fused front end (T <= 16),
    the split top-k (T <= 128) and the standalone router (T > 128)."""
    from vllm_neuron_amd import _lib
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.functional.moe._common import resolve_experts
    from vllm_neuron_amd.functional.moe.moe_block_tkg import block_decode_raw
    from vllm_neuron_amd.weights import MXFP4Experts

    lt = synthetic.layer_tensors(synthetic.GPT_OSS_20B, 65, E=32)
    ref = RefLayer(lt)
    w = MXFP4Experts.from_checkpoint(lt.gate_up_blocks, lt.gate_up_scales, lt.down_blocks,
                                     lt.down_scales, lt.gate_up_bias, lt.down_bias).to(dev)
    ex = resolve_experts(w.gu_q, w.gu_s, w.dn_q, w.dn_s, w.gu_bias, w.dn_bias)
    x = synthetic.tokens(66, T, ref.H)
    rw16 = lt.router_w.to(torch.float16)
    rb16 = synthetic.normal_bf16(67, (32,), 0.5).to(torch.float16)
    gamma = torch.ones(ref.H)
    out, logits, idx = block_decode_raw(
        x.to(dev), gamma.to(dev), 1e-6, None, rw16.T.to(dev), rb16.to(dev), _lib.ROUTER_SOFTMAX,
        False, False, 4, ex, _lib.ACT_SWISH, _lib.clamps_array(None, 7.0, -6.0, 8.0),
        _lib.SCALE_POST, True, want_idx=True)
    from vllm_neuron_amd import functional as NF

    xn = NF.rmsnorm(x.to(dev), gamma.to(dev), 1e-6).cpu()  # the block's RMSNorm kernel
    _norm_stage(xn, x, gamma, 1e-6, ref.H, all_cols=False)
    logits_r = xn.float() @ rw16.T.float() + rb16.float()  # fp32 router of the flow
    top, idx_r = torch.topk(logits_r, 4, dim=1)
    top = torch.softmax(top, dim=1)
    assert torch.allclose(logits.cpu(), logits_r, rtol=1e-5, atol=1e-5)
    ties = check_indices(idx, logits_r, idx_r, 4, f"block decode fp16 router T={T}")
    aff = torch.zeros(T, 32).scatter_(1, idx_r, top)
    want = ref.decode_routed(xn, aff)
    check_close(out.cpu(), want, ties, f"block decode fp16 router T={T}")
