"""Enumerations of the operator API, with the member names the reference uses.

The reference imports these from the external nkilib package
(nkilib.core.utils.common_types, nkilib.core.moe.moe_cte) and defines
RouterComputationOrder in vllm_neuron/functional/moe/router.py:18-69.  Callers
that pass enum members by name keep working unchanged.
"""

from __future__ import annotations

from enum import Enum


class ActFnType(Enum):
    SiLU = "SiLU"
    GELU = "GELU"
    GELU_Tanh_Approx = "GELU_Tanh_Approx"
    Swish = "Swish"


class NormType(Enum):
    NO_NORM = "NO_NORM"
    RMS_NORM = "RMS_NORM"
    RMS_NORM_SKIP_GAMMA = "RMS_NORM_SKIP_GAMMA"
    LAYER_NORM = "LAYER_NORM"


class ExpertAffinityScaleMode(Enum):
    NO_SCALE = "NO_SCALE"
    POST_SCALE = "POST_SCALE"
    PRE_SCALE = "PRE_SCALE"
    PRE_SCALE_DELAYED = "PRE_SCALE_DELAYED"


class RouterActFnType(Enum):
    SOFTMAX = "SOFTMAX"
    SIGMOID = "SIGMOID"


class RouterComputationOrder(Enum):
    PRENORM_LINEAR_TOPK_ACT_SCATTER = "prenorm_linear_topk_act_scatter"
    PRENORM_LINEAR_ACT_TOPK_RENORM_SCATTER = "prenorm_linear_act_topk_renorm_scatter"
    PRENORM_LINEAR_TOPK_SCATTER_ACT = "prenorm_linear_topk_scatter_act"


class MoECTEImplementation(Enum):
    shard_on_block = "shard_on_block"
    shard_on_i = "shard_on_i"
    shard_on_i_hybrid = "shard_on_i_hybrid"
    shard_on_i_dropping = "shard_on_i_dropping"
    shard_on_block_mx = "shard_on_block_mx"
    shard_on_i_mx = "shard_on_i_mx"
    shard_on_i_mx_hybrid = "shard_on_i_mx_hybrid"


class BlockShardStrategy(Enum):
    PING_PONG = "PING_PONG"
    HI_LO = "HI_LO"


class QuantizationType(Enum):
    NONE = "NONE"
    STATIC = "STATIC"
    ROW = "ROW"
    MX = "MX"
    STATIC_MX = "STATIC_MX"


class MoEAllToAllVStrategy(Enum):
    DISABLED = "DISABLED"
    PRESERVE_ROW_ORDER = "PRESERVE_ROW_ORDER"
    PACK_OUTPUT_ROWS = "PACK_OUTPUT_ROWS"


def member_name(v) -> str:
    """Enum member (this module's or any other enum with the same names) or string -> name."""
    return getattr(v, "name", str(v))
