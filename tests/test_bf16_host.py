"""Host-side rules of the bf16 expert-weight path (no GPU needed): which moe_cte
implementations take bf16 weights, and the weight-format constants of the C-ABI."""

import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]


def _cte_args(E=2, H=64, I=64, T=4):
    return dict(hidden_states=torch.zeros(T, H, dtype=torch.bfloat16),
                expert_affinities_masked=torch.zeros(T * E, 1),
                gate_up_proj_weight=torch.zeros(E, H, 2, I, dtype=torch.bfloat16),
                down_proj_weight=torch.zeros(E, I, H, dtype=torch.bfloat16),
                token_position_to_id=torch.zeros(128, dtype=torch.int32),
                block_to_expert=torch.zeros(1, dtype=torch.int32), block_size=128)


@pytest.mark.parametrize("impl", ["shard_on_block_mx", "shard_on_i_mx", "shard_on_i_mx_hybrid"])
def test_mx_implementations_assert_scales_for_bf16_weights(impl):
    """moe_cte.py:596-605: the MX implementations assert that both scales are given."""
    from vllm_neuron_amd import functional as NF
    from vllm_neuron_amd.enums import MoECTEImplementation

    with pytest.raises(AssertionError, match="scale"):
        NF.moe_cte(implementation=getattr(MoECTEImplementation, impl), **_cte_args())


def test_mx_implementation_rejects_bf16_weights_with_scales():
    from vllm_neuron_amd import functional as NF

    s = torch.zeros(2, 4, 128, dtype=torch.uint8)
    with pytest.raises(ValueError, match="packed MX"):
        NF.moe_cte(implementation="shard_on_block_mx", gate_up_proj_scale=s, down_proj_scale=s,
                   **_cte_args())


def test_packed_weights_still_need_scales_under_shard_on_block():
    from vllm_neuron_amd import functional as NF

    a = _cte_args()
    a["gate_up_proj_weight"] = torch.zeros(2, 8, 512, dtype=torch.uint8)
    with pytest.raises(AssertionError, match="scale"):
        NF.moe_cte(implementation="shard_on_block", **a)


def test_weight_format_constants_match_the_header():
    from vllm_neuron_amd import _lib

    hdr = (ROOT / "include" / "mxfp4_moe.h").read_text()
    got = {m.group(1): int(m.group(2))
           for m in re.finditer(r"#define MXMOE_WFMT_(\w+) (\d+)", hdr)}
    assert got == {"MXFP4": _lib.WFMT_MXFP4, "MXFP8": _lib.WFMT_MXFP8, "BF16": _lib.WFMT_BF16}
