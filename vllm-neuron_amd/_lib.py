"""ctypes binding of libmxmoe.so (the C-ABI declared in include/mxfp4_moe.h).

The library is loaded lazily on first use.  There is no fallback: if the built
library is missing, or no GPU is visible, the functional API raises.
"""

from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libmxmoe.so"

ACT_SILU, ACT_GELU, ACT_SWISH = 0, 1, 2
SCALE_POST, SCALE_NO, SCALE_PRE, SCALE_PRE_DELAYED = 0, 1, 2, 3
ROUTER_SOFTMAX, ROUTER_SIGMOID = 0, 1
DT_F32, DT_F16, DT_BF16 = 0, 1, 2
WFMT_MXFP4, WFMT_MXFP8, WFMT_BF16 = 0, 1, 2

_P = C.c_void_p
_I64 = C.c_int64
_I = C.c_int
_F = C.c_float
_SZ = C.c_size_t

# name -> (restype, argtypes)
_SIGNATURES = {
    "mxmoe_version": (_I, []),
    "mxmoe_last_error": (C.c_char_p, []),
    "mxmoe_dequant_bf16": (_I, [_P, _P, _P, _I64, _I64, _P]),
    "mxmoe_dequant_mxfp8_bf16": (_I, [_P, _P, _P, _I64, _I64, _P]),
    "mxmoe_linear": (_I, [_P, _I64, _P, _P, _I, _I64, _I64, _P, _P]),
    "mxmoe_router_workspace_bytes": (_SZ, [_I64, _I64]),
    "mxmoe_router_topk": (_I, [_P, _I, _P, _I, _P, _I, _I64, _I64, _I64, _I, _I, _I, _I, _F, _I,
                               _P, _P, _P, _P, _P, _SZ, _P]),
    "mxmoe_rmsnorm": (_I, [_P, _P, _I64, _I64, _I64, _I, _F, _I, _P, _P]),
    "mxmoe_rmsnorm_router_topk_workspace_bytes": (_SZ, [_I64, _I64, _I]),
    "mxmoe_rmsnorm_router_topk": (_I, [_P, _P, _I64, _F, _P, _I, _P, _I, _I64, _I64, _I64, _I, _I,
                                       _I, _P, _P, _P, _P, _SZ, _P]),
    "mxmoe_blockwise_workspace_bytes": (_SZ, [_I64, _I64]),
    "mxmoe_blockwise_mapping": (_I, [_P, _P, _I64, _I64, _I, _I64, _I64, _P, _P, _P, _P, _P, _P,
                                     _SZ, _P]),
    "mxmoe_moe_cte_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64, _I]),
    "mxmoe_moe_cte": (_I, [_P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _I64, _I64, _I64,
                           _I64, _I64, _I64, _I, _P, _I, _I, _P, _P, _SZ, _P, _P]),
    "mxmoe_moe_prefill_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I, _I64]),
    "mxmoe_moe_prefill": (_I, [_P, _P, _I, _P, _I, _I, _I, _I, _F, _I, _P, _P, _P, _P, _P, _I, _P,
                               _P, _I64, _I64, _I64, _I64, _I, _I64, _I, _P, _I, _P, _P, _SZ, _P,
                               _P]),
    "mxmoe_moe_tkg_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I]),
    "mxmoe_moe_tkg": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _I, _P,
                           _I, _P, _P, _SZ, _P, _P]),
    "mxmoe_moe_tkg_bf16_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I]),
    "mxmoe_moe_tkg_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _I, _P,
                                _I, _P, _P, _SZ, _P]),
    "mxmoe_moe_decode_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I]),
    "mxmoe_moe_decode": (_I, [_P, _P, _I, _P, _I, _I, _I, _I, _F, _P, _P, _P, _P, _P, _P, _I64,
                              _I64, _I64, _I64, _I, _I, _P, _I, _P, _P, _P, _P, _SZ, _P, _P]),
    "mxmoe_moe_block_decode_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I]),
    "mxmoe_moe_block_decode": (_I, [_P, _P, _I64, _F, _P, _I, _P, _I, _I, _I, _I, _F, _P, _P, _P,
                                    _P, _P, _P, _I64, _I64, _I64, _I64, _I, _I, _P, _I, _P, _P,
                                    _P, _P, _SZ, _P, _P]),
    "mxmoe_moe_block_decode_noalloc": (_I, [_P, _P, _I64, _F, _P, _I, _P, _I, _I, _I, _I, _F, _P,
                                            _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _I,
                                            _P, _I, _P, _P, _P, _P, _P]),
    "mxmoe_probe_hw_dequant": (_I, [_P, _P, _P, _I64, _I64, _P]),
    "mxmoe_probe_hw_dequant_fp8": (_I, [_P, _P, _P, _I64, _I64, _P]),
    "mxmoe_probe_mfma": (_I, [_P, _P, _P, _P]),
}

_lib = None
_lock = threading.Lock()


class MXMoEError(RuntimeError):
    """A C-ABI entry point returned an error status."""


def load_library(path: Path = LIB_PATH):
    """Load and bind the shared library (no GPU is touched)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not path.exists():
            raise RuntimeError(
                f"MI355X MoE extension not built: {path} is missing "
                "(run python vllm-neuron_amd/build_lib.py)")
        lib = C.CDLL(str(path))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def lib():
    return _lib if _lib is not None else load_library()


def exported_symbols():
    return list(_SIGNATURES)


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().mxmoe_last_error().decode(errors="replace")
        raise MXMoEError(f"{what} failed ({rc}): {msg}")


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def require_cuda(*tensors) -> torch.device:
    """All tensors on one GPU; returns it.  No CPU path exists."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("the MI355X MoE kernels need GPU tensors; got a CPU tensor")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError("tensors are on different devices")
    if dev is None:
        raise RuntimeError("no tensor given")
    return dev


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def event_array(events):
    """torch.cuda.Event list -> a C array of their hipEvent_t handles (or None)."""
    if not events:
        return None
    for e in events:
        if not e.cuda_event:  # torch creates the HIP event on its first record
            e.record()
    return (C.c_void_p * len(events))(*[e.cuda_event for e in events])


_TORCH_DT = {torch.float32: DT_F32, torch.float16: DT_F16, torch.bfloat16: DT_BF16}


def dtype_code(dt: torch.dtype, what: str, allowed=(torch.float32, torch.float16,
                                                    torch.bfloat16)) -> int:
    """torch dtype -> MXMOE_DT_* code; NotImplementedError for any other dtype."""
    if dt not in allowed:
        names = ", ".join(str(a).replace("torch.", "") for a in allowed)
        raise NotImplementedError(f"{what} must be one of {names}, got {dt}")
    return _TORCH_DT[dt]


def clamps_array(gate_lo, gate_hi, up_lo, up_hi):
    inf = float("inf")
    vals = [(-inf if gate_lo is None else float(gate_lo)), (inf if gate_hi is None else float(gate_hi)),
            (-inf if up_lo is None else float(up_lo)), (inf if up_hi is None else float(up_hi))]
    return (C.c_float * 4)(*vals)
