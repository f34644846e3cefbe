"""The functional API's error conventions, on the CPU: the exception type the reference
raises for each misuse, raised before any GPU work (vllm_neuron/functional error
conventions: ValueError for shape and range validation, NotImplementedError for what has
no kernel, AssertionError for missing MX scales, RuntimeError for MX compute on the CPU).
"""

import pytest
import torch

from vllm_neuron_amd import functional as NF
from vllm_neuron_amd.enums import (ExpertAffinityScaleMode, MoEAllToAllVStrategy,
                                   MoECTEImplementation, QuantizationType,
                                   RouterComputationOrder)

T, H, E, K = 4, 64, 8, 2


def _x():
    return torch.zeros(T, H, dtype=torch.bfloat16)


def _w():
    return torch.zeros(H, E, dtype=torch.bfloat16)


# router.py:631-677 (_validate_router_inputs): every case is a ValueError.
@pytest.mark.parametrize("case", [
    "hidden_3d", "weights_1d", "hidden_mismatch", "bias_shape", "gamma_shape", "top_k_0",
    "top_k_above_e", "computation_dtype", "order_not_enum"])
def test_router_input_validation(case):
    x, w, kw, k = _x(), _w(), {}, K
    if case == "hidden_3d":
        x = x.view(1, T, H)
    elif case == "weights_1d":
        w = w.reshape(-1)
    elif case == "hidden_mismatch":
        w = torch.zeros(H + 32, E, dtype=torch.bfloat16)
    elif case == "bias_shape":
        kw["router_bias"] = torch.zeros(E + 1, dtype=torch.bfloat16)
    elif case == "gamma_shape":
        kw["gamma"] = torch.zeros(H - 1, dtype=torch.bfloat16)
    elif case == "top_k_0":
        k = 0
    elif case == "top_k_above_e":
        k = E + 1
    elif case == "computation_dtype":
        kw["computation_dtype"] = torch.int32
    elif case == "order_not_enum":
        kw["router_computation_order"] = "PRENORM_LINEAR_TOPK_ACT_SCATTER"
    with pytest.raises(ValueError):
        NF.router(x, w, k, **kw)


def test_router_activation_errors():
    """router.py:568-598: an unknown activation name is a ValueError; a callable
    activation has no kernel here (NotImplementedError); valid inputs on CPU tensors reach
    the device check (RuntimeError), as the reference's MX paths do on the CPU."""
    with pytest.raises(ValueError):
        NF.router(_x(), _w(), K, activation="relu")
    with pytest.raises(NotImplementedError):
        NF.router(_x(), _w(), K, activation=torch.sigmoid)
    for act in ("softmax", "sigmoid"):
        with pytest.raises(RuntimeError, match="GPU"):
            NF.router(_x(), _w(), K, activation=act,
                      router_computation_order=RouterComputationOrder.PRENORM_LINEAR_TOPK_ACT_SCATTER)


def test_blockwise_mapping_errors():
    """moe_blockwise.py:24-156: tensor-parallel mapping needs several GPUs; an affinity
    matrix whose width is not num_local_experts is rejected before any device work."""
    aff = torch.zeros(T, E)
    with pytest.raises(NotImplementedError):
        NF.build_blockwise_mapping(aff, E, K, 256, tp_degree=2)
    with pytest.raises(ValueError):
        NF.build_blockwise_mapping(aff[:, :E - 1], E, K, 256)
    with pytest.raises(RuntimeError, match="GPU"):
        NF.build_blockwise_mapping(aff, E, K, 256)


def _cte_args(I=256):
    # packed MXFP4 experts: gate_up [E, 2I/16, 8H] and down [E, H/16, 8I] uint8
    gu = torch.zeros(E, 2 * I // 16, 8 * H, dtype=torch.uint8)
    dn = torch.zeros(E, H // 16, 8 * I, dtype=torch.uint8)
    aff = torch.zeros(T * E, 1)
    tp2id = torch.full((256,), -1, dtype=torch.int32)
    b2e = torch.zeros(1, dtype=torch.int32)
    return (_x(), aff, gu, dn, tp2id, b2e, 256)


def test_moe_cte_errors():
    """moe_cte.py:584-615 (_can_use_moe_cte_kernel): the MX implementations assert both
    scales, and MX compute on the CPU is a RuntimeError; STATIC_MX (:282-345) and output
    dtypes other than bf16 / fp32 have no kernel here (NotImplementedError)."""
    args = _cte_args()
    gu_s = torch.zeros(E, 2 * 256 // 64, 2 * H, dtype=torch.uint8)
    dn_s = torch.zeros(E, H // 64, 2 * 256, dtype=torch.uint8)
    with pytest.raises(AssertionError):
        NF.moe_cte(*args, implementation=MoECTEImplementation.shard_on_block_mx,
                   gate_up_proj_scale=None, down_proj_scale=dn_s)
    with pytest.raises(RuntimeError, match="GPU"):
        NF.moe_cte(*args, implementation=MoECTEImplementation.shard_on_block_mx,
                   gate_up_proj_scale=gu_s, down_proj_scale=dn_s)
    with pytest.raises(NotImplementedError):
        NF.moe_cte(*args, gate_up_proj_scale=gu_s, down_proj_scale=dn_s,
                   quantization_type=QuantizationType.STATIC_MX)
    with pytest.raises(NotImplementedError):
        NF.moe_cte(*args, gate_up_proj_scale=gu_s, down_proj_scale=dn_s,
                   output_dtype=torch.float16)
    with pytest.raises(NotImplementedError):
        NF.moe_cte(*args, gate_up_proj_scale=gu_s, down_proj_scale=dn_s,
                   down_activations=torch.zeros(1))


def test_moe_tkg_errors():
    """moe_tkg.py:191-194: anything but MXFP4 weights raises NotImplementedError (there is
    no CPU flow for this op); the all-to-all-v packed inputs need several GPUs and FP8
    activation quantization has no kernel here."""
    x = _x()
    gu = torch.zeros(E, 2 * 256 // 16, 8 * H, dtype=torch.uint8)
    dn = torch.zeros(E, H // 16, 8 * 256, dtype=torch.uint8)
    aff = torch.zeros(T, E)
    idx = torch.zeros(T, K, dtype=torch.int32)
    with pytest.raises(NotImplementedError):
        NF.moe_tkg(x, gu.to(torch.bfloat16), dn.to(torch.bfloat16), aff, idx, False)
    with pytest.raises(NotImplementedError):
        NF.moe_tkg(x, gu, dn, aff, idx, False,
                   all_to_all_v_strategy=MoEAllToAllVStrategy.PRESERVE_ROW_ORDER)
    with pytest.raises(NotImplementedError):
        NF.moe_tkg(x, gu, dn, aff, idx, False, hidden_input_scale=torch.ones(1))
    with pytest.raises(ValueError):
        NF.moe_tkg(x, gu, dn, None, idx, False)


def test_moe_block_tkg_errors():
    """moe_block_tkg.py:520-545: shared experts and the fused residual add raise
    NotImplementedError, before any device work."""
    inp = torch.zeros(1, T, H, dtype=torch.bfloat16)
    gamma = torch.ones(1, H, dtype=torch.bfloat16)
    gu = torch.zeros(E, 2 * 256 // 16, 8 * H, dtype=torch.uint8)
    dn = torch.zeros(E, H // 16, 8 * 256, dtype=torch.uint8)
    with pytest.raises(NotImplementedError):
        NF.moe_block_tkg(inp, gamma, _w(), gu, dn, None, K,
                         shared_expert_gate_w=torch.zeros(1))
    with pytest.raises(NotImplementedError):
        NF.moe_block_tkg(inp, gamma, _w(), gu, dn, None, K, residual=torch.zeros(1))


def test_scale_mode_names_follow_the_reference_enum():
    """Scaling modes are taken by enum member or name, as the reference passes them."""
    assert {m.name for m in ExpertAffinityScaleMode} >= {"NO_SCALE", "POST_SCALE",
                                                         "PRE_SCALE", "PRE_SCALE_DELAYED"}
