"""MoE operators (vllm_neuron/functional/moe counterparts)."""

from .moe_block_tkg import moe_block_tkg, rmsnorm
from .moe_blockwise import build_blockwise_mapping, num_blocks
from .moe_cte import moe_cte
from .moe_tkg import moe_tkg
from .rmsnorm_router_topk_tkg import rmsnorm_router_topk_tkg
from .router import router

__all__ = ["router", "build_blockwise_mapping", "num_blocks", "moe_cte", "moe_tkg",
           "moe_block_tkg", "rmsnorm", "rmsnorm_router_topk_tkg"]
