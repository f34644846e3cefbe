"""MI355X-native MXFP4 mixture-of-experts expert path.

Drop-in counterpart of the MoE/MXFP4 operators of vllm-neuron's
``vllm_neuron.functional``: router top-k, blockwise token -> expert mapping, prefill
expert MLP (moe_cte), decode expert MLP (moe_tkg / moe_block_tkg) and MXFP4
dequantization, all running hand-written gfx950 HIP kernels from libmxmoe.so.
"""

from . import checkpoint, enums, functional, neuron_layout, weights  # noqa: F401
from ._lib import MXMoEError, load_library  # noqa: F401

__version__ = "0.1.0"
