"""Operator API of the MXFP4 MoE path, with the names of vllm_neuron.functional
(vllm_neuron/functional/__init__.py:23-33, __all__ :42-74) for the MoE entries and the
dense MX mlp."""

from ..enums import (ActFnType, ExpertAffinityScaleMode, MoECTEImplementation, NormType,
                     QuantizationType, RouterActFnType, RouterComputationOrder)
from .mlp import mlp
from .moe import (build_blockwise_mapping, moe_block_tkg, moe_cte, moe_tkg, num_blocks, rmsnorm,
                  rmsnorm_router_topk_tkg, router)
from .mxfp4 import (dequantize_mxfp4_to_bf16, dequantize_mxfp8_to_bf16, mxfp4_linear,
                    mxfp8_linear)

__all__ = [
    "router", "build_blockwise_mapping", "moe_cte", "moe_tkg", "moe_block_tkg", "rmsnorm",
    "rmsnorm_router_topk_tkg", "num_blocks", "dequantize_mxfp4_to_bf16", "mxfp4_linear",
    "dequantize_mxfp8_to_bf16", "mxfp8_linear", "mlp",
    "ActFnType", "ExpertAffinityScaleMode", "MoECTEImplementation", "NormType", "QuantizationType",
    "RouterActFnType", "RouterComputationOrder",
]
