"""The C-ABI library loads, exports every symbol the header declares, and rejects bad
arguments with its documented status codes (no GPU work is issued by these calls)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mxfp4_moe.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(mxmoe_\w+)\(", text, re.M)))


def test_header_and_binding_agree():
    from vllm_neuron_amd import _lib

    assert declared_functions() == sorted(_lib.exported_symbols())


def test_library_exports_every_declared_symbol():
    from vllm_neuron_amd import _lib

    lib = _lib.load_library()
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in declared_functions():
        assert hasattr(raw, name), name
    assert lib.mxmoe_version() >= 100


def test_argument_errors_are_reported():
    from vllm_neuron_amd import _lib

    lib = _lib.load_library()
    dummy = ctypes.c_void_p(16)
    rc = lib.mxmoe_dequant_bf16(dummy, dummy, dummy, 4, 31, None)
    assert rc == -1 and b"multiple of 32" in lib.mxmoe_last_error()
    rc = lib.mxmoe_router_topk(dummy, dummy, None, 4, 64, 8, 9, 0, 0, 0, 0.0, dummy, dummy, dummy,
                               dummy, None, 0, None)
    assert rc == -1 and b"top_k" in lib.mxmoe_last_error()
    rc = lib.mxmoe_blockwise_mapping(dummy, None, 100, 8, 2, 64, 3, dummy, dummy, dummy, dummy,
                                     None, dummy, 1 << 20, None)
    assert rc == -1 and b"n_blocks" in lib.mxmoe_last_error()
    rc = lib.mxmoe_moe_cte(dummy, dummy, dummy, dummy, dummy, dummy, None, None, dummy, dummy, 4,
                           100, 64, 2880, 2880, 8, 2, None, 0, 0, dummy, dummy, 1 << 30, None,
                           None)
    assert rc == -1 and b"block_size" in lib.mxmoe_last_error()
    rc = lib.mxmoe_moe_tkg(dummy, dummy, dummy, dummy, dummy, dummy, dummy, None, None, 4, 2880,
                           2880, 32, 4, 2, None, 0, dummy, dummy, 10, None, None)
    assert rc == -3 and b"workspace" in lib.mxmoe_last_error()


def test_workspace_queries():
    from vllm_neuron_amd import _lib

    lib = _lib.load_library()
    n = lib.mxmoe_moe_cte_workspace_bytes(4096, 2880, 2880, 128, 256, 191)
    assert n >= 191 * 256 * 2880 * 2 * 2 + 4096 * 128 * 4
    assert lib.mxmoe_moe_tkg_workspace_bytes(64, 2880, 2880, 128, 4) >= 256 * 2880 * 8


def test_functional_api_refuses_cpu_tensors():
    import torch

    from vllm_neuron_amd import functional as NF

    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    w = torch.zeros(64, 8, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        NF.router(x, w, 2)
    with pytest.raises(ValueError):
        NF.router(x, w, 9)
