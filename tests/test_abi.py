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
    rc = lib.mxmoe_router_topk(dummy, 2, dummy, 2, None, 2, 4, 64, 8, 9, 0, 0, 0, 0.0, 0, dummy,
                               dummy, dummy, dummy, None, 0, None)
    assert rc == -1 and b"top_k" in lib.mxmoe_last_error()
    # fp32 computation needs bf16 activations (every product exact)
    rc = lib.mxmoe_router_topk(dummy, 1, dummy, 2, None, 2, 4, 64, 8, 2, 0, 0, 0, 0.0, 0, dummy,
                               dummy, dummy, dummy, None, 0, None)
    assert rc == -1 and b"bf16 activations" in lib.mxmoe_last_error()
    rc = lib.mxmoe_rmsnorm_router_topk(dummy, dummy, 64, 1e-6, dummy, 1, None, 1, 4, 64, 8, 2, 0,
                                       0, dummy, dummy, dummy, dummy, 1 << 20, None)
    assert rc == -1 and b"matmul dtype" in lib.mxmoe_last_error()
    rc = lib.mxmoe_rmsnorm(dummy, dummy, 4, 64, 65, 0, 1e-6, 2, dummy, None)
    assert rc == -1 and b"bad shape" in lib.mxmoe_last_error()
    rc = lib.mxmoe_blockwise_mapping(dummy, None, 100, 8, 2, 64, 3, dummy, dummy, dummy, dummy,
                                     None, dummy, 1 << 20, None)
    assert rc == -1 and b"n_blocks" in lib.mxmoe_last_error()
    rc = lib.mxmoe_moe_cte(dummy, dummy, dummy, dummy, dummy, dummy, 0, None, None, None, dummy,
                           dummy, 4, 100, 64, 2880, 2880, 8, 2, None, 0, 0, dummy, dummy, 1 << 30,
                           None, None)
    assert rc == -1 and b"block_size" in lib.mxmoe_last_error()
    rc = lib.mxmoe_moe_cte(dummy, dummy, dummy, dummy, dummy, dummy, 3, None, None, None, dummy,
                           dummy, 4, 256, 64, 2880, 2880, 8, 2, None, 0, 0, dummy, dummy, 1 << 30,
                           None, None)
    assert rc == -1 and b"weight format" in lib.mxmoe_last_error()
    # bf16 weights: no scales needed, rows read 16 bytes at a time
    odd = ctypes.c_void_p(18)
    rc = lib.mxmoe_moe_cte(dummy, dummy, odd, None, dummy, None, 2, None, None, None, dummy,
                           dummy, 4, 256, 64, 2880, 2880, 8, 2, None, 0, 0, dummy, dummy, 1 << 30,
                           None, None)
    assert rc == -1 and b"16-byte aligned" in lib.mxmoe_last_error()
    rc = lib.mxmoe_moe_cte(dummy, dummy, dummy, None, dummy, None, 0, None, None, None, dummy,
                           dummy, 4, 256, 64, 2880, 2880, 8, 2, None, 0, 0, dummy, dummy, 1 << 30,
                           None, None)
    assert rc == -1 and b"null pointer" in lib.mxmoe_last_error()
    rc = lib.mxmoe_linear(dummy, 4, dummy, dummy, 5, 64, 64, dummy, None)
    assert rc == -1 and b"weight format" in lib.mxmoe_last_error()
    rc = lib.mxmoe_dequant_mxfp8_bf16(dummy, dummy, dummy, 4, 48, None)
    assert rc == -1 and b"multiple of 32" in lib.mxmoe_last_error()
    # 32-bit activation-row offsets: slots x columns must stay below 4 GiB
    rc = lib.mxmoe_moe_cte(dummy, dummy, dummy, dummy, dummy, dummy, 0, None, None, None, dummy,
                           dummy, 2048, 256, 64, 8192, 8192, 8, 2, None, 0, 0, dummy, dummy,
                           1 << 40, None, None)
    assert rc == -1 and b"4 GiB" in lib.mxmoe_last_error()
    rc = lib.mxmoe_moe_tkg(dummy, dummy, dummy, dummy, dummy, dummy, dummy, None, None, 4, 2880,
                           2880, 32, 4, 2, None, 0, dummy, dummy, 10, None, None)
    assert rc == -3 and b"workspace" in lib.mxmoe_last_error()


def test_workspace_queries():
    from vllm_neuron_amd import _lib

    lib = _lib.load_library()
    n = lib.mxmoe_moe_cte_workspace_bytes(4096, 2880, 2880, 128, 256, 191, 0)
    assert n >= 191 * 256 * 2880 * 2 * 2 + 4096 * 128 * 4
    n_pre = lib.mxmoe_moe_cte_workspace_bytes(4096, 2880, 2880, 128, 256, 191, 2)
    assert n_pre >= n + 191 * 256 * 2880 * 2  # the scaled rows of PRE_SCALE
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


def test_packed_bias_shapes_are_strict():
    """Biases of packed experts take [E, 2, I] / [E, 2I] and [E, H] / [E, 1, H] only; the
    reference's 5-D kernel-layout bias view (model_mxfp4.py:1195-1201) raises instead of
    being reinterpreted."""
    import torch

    from vllm_neuron_amd.functional.moe._common import down_bias, gate_up_bias

    E, I, H = 4, 3072, 3072
    assert gate_up_bias(torch.zeros(E, 2 * I, dtype=torch.bfloat16), E, I).shape == (E, 2, I)
    assert gate_up_bias(torch.zeros(E, 2, I, dtype=torch.bfloat16), E, I).shape == (E, 2, I)
    with pytest.raises(ValueError):
        gate_up_bias(torch.zeros(E, 2 * I, dtype=torch.bfloat16).view(E, 128, 2, 6, 4), E, I)
    with pytest.raises(ValueError):
        gate_up_bias(torch.zeros(E, I, 2, dtype=torch.bfloat16), E, I)
    assert down_bias(torch.zeros(E, 1, H, dtype=torch.bfloat16), E, H).shape == (E, H)
    with pytest.raises(ValueError):
        down_bias(torch.zeros(E * H, dtype=torch.bfloat16), E, H)


def test_derived_cache_never_aliases_freed_storage():
    """A cached transposed router weight belongs to its source tensor: a new tensor at a
    reused address, an in-place update and an inference tensor all get fresh results."""
    import gc

    import torch

    from vllm_neuron_amd.functional.moe import _cache

    _cache.clear()
    calls = []

    def make(t):
        calls.append(1)
        return t.t().contiguous() * 1

    a = torch.randn(8, 6)
    r1 = _cache.derived("t", (a,), lambda: make(a))
    assert _cache.derived("t", (a,), lambda: make(a)) is r1 and len(calls) == 1
    a.add_(1.0)  # in-place update: version bump
    r2 = _cache.derived("t", (a,), lambda: make(a))
    assert len(calls) == 2 and torch.equal(r2, a.t())
    ptr = a.data_ptr()
    del a, r1, r2
    gc.collect()
    hits = 0
    for _ in range(20):  # the allocator usually hands the same block to the next tensor
        b = torch.full((8, 6), 3.0)
        hits += b.data_ptr() == ptr
        rb = _cache.derived("t", (b,), lambda: make(b))
        assert torch.equal(rb, b.t())
        del b, rb
        gc.collect()
    print("address reused", hits, "times")
    with torch.inference_mode():
        c = torch.randn(8, 6)
    n = len(calls)
    _cache.derived("t", (c,), lambda: make(c))
    _cache.derived("t", (c,), lambda: make(c))
    assert len(calls) == n + 2  # inference tensors are never cached
    v = torch.randn(6, 8)
    assert _cache.transposed_rows(v.t()).data_ptr() == v.data_ptr()  # [E, H] storage: a view


def test_derived_cache_releases_freed_sources():
    """An entry never keeps its sources alive: freeing the key frees the entry and its
    converted copy, a freed second input makes the entry stale, and a value that is a
    view of the key is returned uncached (it would pin the key)."""
    import gc
    import weakref

    import torch

    from vllm_neuron_amd.functional.moe import _cache

    _cache.clear()
    src = torch.randn(64, 32)
    other = torch.randn(32)
    val = _cache.derived("conv", (src, other), lambda: src.t().contiguous() + other[:1])
    assert _cache.derived("conv", (src, other), lambda: 1 / 0) is val  # a hit
    assert _cache.entries() == 1
    w_src, w_val = weakref.ref(src), weakref.ref(val)
    del src, val
    gc.collect()
    assert w_src() is None and w_val() is None  # source and converted copy released
    assert _cache.entries() == 0

    key = torch.randn(16, 8)
    b = torch.randn(8)
    r1 = _cache.derived("sum", (key, b), lambda: key + b)
    w_b = weakref.ref(b)
    del b
    gc.collect()
    assert w_b() is None  # the entry does not hold its second input
    b2 = torch.randn(8)
    r2 = _cache.derived("sum", (key, b2), lambda: key + b2)
    assert r2 is not r1 and torch.equal(r2, key + b2)

    k2 = torch.randn(4, 4)
    v1 = _cache.derived("view", (k2,), lambda: k2.view(16))
    v2 = _cache.derived("view", (k2,), lambda: k2.view(16))
    assert v1 is not v2  # a view of the key is not cached
    w_k2 = weakref.ref(k2)
    del k2, v1, v2
    gc.collect()
    assert w_k2() is None
    del key, b2, r1, r2
    gc.collect()
    assert _cache.entries() == 0


def test_moe_cte_no_scale_is_accepted():
    """NO_SCALE passes the mode check (it runs on the GPU: here the CPU tensors stop it)."""
    import torch

    from vllm_neuron_amd import functional as NF

    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU tensors"):
        NF.moe_cte(x, torch.zeros(8, 1), torch.zeros(2, 8, 512, dtype=torch.uint8),
                   torch.zeros(2, 4, 256, dtype=torch.uint8), torch.zeros(256, dtype=torch.int32),
                   torch.zeros(1, dtype=torch.int32), 256,
                   gate_up_proj_scale=torch.zeros(2, 1, 128, dtype=torch.uint8),
                   down_proj_scale=torch.zeros(2, 1, 128, dtype=torch.uint8),
                   expert_affinities_scaling_mode="NO_SCALE")
