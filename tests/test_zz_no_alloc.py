"""mxmoe_moe_block_decode_noalloc: the decode block over the library's own scratch array.

Checked through the C-ABI against mxmoe_moe_block_decode with a caller workspace on the
same inputs: the kernels are deterministic, so output, logits and selected experts must
be bit-identical.  Two calls in a row, the second smaller, share the array (stale
contents of the first call must not leak into the second).  The size limit is a host
check and is tested without a GPU.
"""

import pytest
import torch



def _layer(dev):
    from vllm_neuron_amd import synthetic
    from vllm_neuron_amd.weights import MXFP4Experts

    lt = synthetic.layer_tensors(synthetic.GPT_OSS_20B, 91)
    w = MXFP4Experts.from_checkpoint(lt.gate_up_blocks, lt.gate_up_scales, lt.down_blocks,
                                     lt.down_scales, lt.gate_up_bias, lt.down_bias).to(dev)
    return lt, w


def _run(noalloc, x, gamma, rw, rb, w, dev):
    from vllm_neuron_amd import _lib

    L = _lib.lib()
    T, H = x.shape
    E, I, K = w.E, w.I, 4
    out = torch.full((T, H), -1, dtype=torch.bfloat16, device=dev)
    logits = torch.full((T, E), -1.0, dtype=torch.float32, device=dev)
    idx = torch.full((T, K), -1, dtype=torch.int32, device=dev)
    clamps = _lib.clamps_array(None, 7.0, -6.0, 8.0)
    common = (x.data_ptr(), gamma.data_ptr(), H, 1e-5, rw.data_ptr(), _lib.DT_BF16,
              rb.data_ptr(), _lib.DT_BF16, _lib.ROUTER_SOFTMAX, 0, 0, 0.0, w.gu_q.data_ptr(),
              w.gu_s.data_ptr(), w.dn_q.data_ptr(), w.dn_s.data_ptr(), w.gu_bias.data_ptr(),
              w.dn_bias.data_ptr(), T, H, I, E, K, _lib.ACT_SWISH, clamps, _lib.SCALE_POST,
              out.data_ptr(), logits.data_ptr(), idx.data_ptr())
    stream = _lib.stream_handle(dev)
    if noalloc:
        rc = L.mxmoe_moe_block_decode_noalloc(*common, None, stream)
        _lib.check(rc, "mxmoe_moe_block_decode_noalloc")
    else:
        ws = _lib.workspace(L.mxmoe_moe_block_decode_workspace_bytes(T, H, I, E, K), dev)
        rc = L.mxmoe_moe_block_decode(*common, ws.data_ptr(), ws.numel(), None, stream)
        _lib.check(rc, "mxmoe_moe_block_decode")
    torch.cuda.synchronize()
    return out.cpu(), logits.cpu(), idx.cpu()


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point(dev):
    from vllm_neuron_amd import synthetic

    lt, w = _layer(dev)
    H = w.H
    gamma = (1.0 + 0.1 * torch.randn(H, generator=torch.Generator().manual_seed(92))).to(dev)
    rw = lt.router_w.to(dev).contiguous()
    rb = synthetic.normal_bf16(93, (w.E,), 0.5).to(dev)
    for T in (64, 16):  # the second call is smaller and reuses the same scratch array
        x = synthetic.tokens(94 + T, T, H).to(dev)
        ref = _run(False, x, gamma, rw, rb, w, dev)
        got = _run(True, x, gamma, rw, rb, w, dev)
        for name, a, b in zip(("output", "logits", "selected experts"), got, ref):
            assert torch.equal(a, b), f"T={T}: {name} differ"
        assert bool((got[2] >= 0).all()) and float(got[0].float().abs().max()) > 0
        print(f"T={T}: no-allocation call bit-identical to the workspace call")


def test_noalloc_rejects_shapes_beyond_its_scratch():
    """The size check runs on the host before anything touches a GPU."""
    from vllm_neuron_amd import _lib

    L = _lib.load_library()
    dummy = 16
    T, H, I, E, K = 1024, 7168, 2048, 256, 8
    need = L.mxmoe_moe_block_decode_workspace_bytes(T, H, I, E, K)
    assert need > (48 << 20)
    args = [dummy, dummy, H, 1e-6, dummy, _lib.DT_BF16, None, _lib.DT_BF16, 0, 0, 0, 0.0, dummy,
            dummy, dummy, dummy, None, None, T, H, I, E, K, _lib.ACT_SILU, None, _lib.SCALE_POST,
            dummy, None, None, None, None]
    rc = L.mxmoe_moe_block_decode_noalloc(*args)
    assert rc == -3 and b"no-allocation entry point holds" in L.mxmoe_last_error()
