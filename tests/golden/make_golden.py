"""Writes the golden fixtures of this directory (run from the repository root:
``python tests/golden/make_golden.py``).

Every fixture is data only (numpy ``.npz`` without object arrays, or JSON): inputs
and the expected outputs.  Expected outputs come from the oracle (the CPU
restatement of the reference path), and each is cross-checked here against an
independent closed form before it is written:

  dequant_kat.npz     all 256 E8M0 scales x 16 e2m1 codes -> bf16 bits; the code
                      table is the reference's FP4 LUT
                      (vllm_neuron/model/gpt_oss/weight_loaders_bf16.py:281-302),
                      checked against the e2m1 definition and float64 ldexp.
  packed_layout.npz   checkpoint blocks/scales of a [80, 320] matrix and their
                      packed bytes (the layout the GPU kernels address), checked
                      element by element against the documented addressing.
  blockwise.npz       build_blockwise_mapping outputs for small cases
                      (vllm_neuron/functional/moe/moe_blockwise.py:24-156), checked
                      against the plain-loop restatement of the closed form.
  router.npz          tie-free router case (router.py:383-440): logits, top-k ids and
                      softmax values, checked against a float64 brute force.
  tiny_layer.npz      a 4-expert MXFP4 layer (H = I = 64, top-2) with 5 tokens:
                      checkpoint tensors, the decode output (fp32 flow of
                      moe_block_tkg.py:223-297) and the prefill output (bf16 flow of
                      moe_cte.py:448-581), checked against a float64 closed form.
  synthetic_sha256.json  SHA-256 of the synthetic generator's tensors for the
                      shapes the tests and the benchmark use, so a run on another
                      host can confirm it generated the same inputs.
"""

from __future__ import annotations

import json
import math
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

import pkgload  # noqa: E402

pkgload.load()
from vllm_neuron_amd import synthetic  # noqa: E402
from vllm_neuron_amd.weights import pack_mxfp4  # noqa: E402

from oracle import blockwise as ob  # noqa: E402
from oracle import mxfp4 as om  # noqa: E402
from oracle import router as orr  # noqa: E402
from oracle.layer import RefLayer  # noqa: E402

REF_FP4_LUT = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
               -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def _e2m1(code: int) -> float:
    s = -1.0 if code & 8 else 1.0
    e, m = (code >> 1) & 3, code & 1
    return s * (m * 0.5) if e == 0 else s * 2.0 ** (e - 1) * (1.0 + m * 0.5)


def _bf16_bits(x: float) -> int:
    """float64 -> float32 (RNE) -> bf16 bits (RNE); NaN -> 0xFFFF."""
    if math.isnan(x):
        return 0xFFFF
    with np.errstate(over="ignore"):  # |x| >= 2^128 becomes +-inf, as in float32
        f = np.array([x], dtype=np.float64).astype(np.float32)
    u = int(f.view(np.uint32)[0])
    if (u & 0x7F800000) == 0x7F800000:
        return u >> 16
    return ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF) >> 16


def dequant_kat():
    codes = np.arange(32) % 16
    byte = (codes[0::2] | (codes[1::2] << 4)).astype(np.uint8)
    blocks = np.tile(byte, (256, 1)).reshape(256, 1, 16)
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    out = om.dequantize_mxfp4_to_bf16(torch.from_numpy(blocks), torch.from_numpy(scales))
    bits = out.view(torch.int16).numpy().astype(np.uint16).reshape(256, 32)
    for c in range(16):
        assert om.FP4_VALUES[c] == REF_FP4_LUT[c] == _e2m1(c)
    for s in range(256):
        for k in range(32):
            v = _e2m1(int(codes[k]))
            if s == 255:
                want = 0xFFFF if v == 0 else (0xFF80 if codes[k] & 8 else 0x7F80)
            elif v == 0:
                want = 0x8000 if codes[k] & 8 else 0
            else:
                want = _bf16_bits(math.ldexp(v, s - 127))
            assert bits[s, k] == want, (s, k, bits[s, k], want)
    np.savez(HERE / "dequant_kat.npz", blocks=blocks, scales=scales, bf16_bits=bits,
             fp4_lut=np.array(REF_FP4_LUT, dtype=np.float32))


def packed_layout():
    g = torch.Generator().manual_seed(7)
    N, K = 80, 320
    blocks = torch.randint(0, 256, (N, K // 32, 16), generator=g, dtype=torch.uint8)
    scales = torch.randint(0, 256, (N, K // 32), generator=g, dtype=torch.uint8)
    d, s = pack_mxfp4(blocks, scales)
    for rg in range(N // 16):
        q, r = divmod(rg, 4)
        for c in range((K + 127) // 128):
            for l in range(64):
                row, kb = 16 * rg + l % 16, 4 * c + l // 16
                if kb >= K // 32:
                    continue
                o = c * 1024 + l * 16
                assert torch.equal(d[rg, o:o + 16], blocks[row, kb])
                assert s[q, c * 256 + 4 * l + r] == scales[row, kb]
    np.savez(HERE / "packed_layout.npz", blocks=blocks.numpy(), scales=scales.numpy(),
             packed_data=d.numpy(), packed_scales=s.numpy())


BLOCKWISE_CASES = [  # T, E, K, B, seed, zipf
    (7, 4, 2, 128, 1, None),
    (37, 8, 2, 128, 2, None),
    (300, 16, 4, 256, 3, 1.2),
    (64, 32, 4, 256, 4, None),
    (5, 3, 3, 128, 5, None),
]


def _routing_affinities(T, E, K, seed, zipf):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, E, generator=g, dtype=torch.float64)
    if zipf:
        logits = logits + synthetic.zipf_bias(seed, E, zipf).double()
    top = torch.topk(logits, K, dim=1)
    aff = torch.zeros(T, E, dtype=torch.float32)
    aff.scatter_(1, top.indices, torch.softmax(top.values, 1).float())
    return aff


def blockwise():
    arrays = {}
    for i, (T, E, K, B, seed, zipf) in enumerate(BLOCKWISE_CASES):
        aff = _routing_affinities(T, E, K, seed, zipf)
        am, tp, b2e, cond = ob.build_blockwise_mapping(aff, E, K, B)
        ltp, lb2e, lcond = ob.build_blockwise_mapping_loops(aff, E, K, B)
        assert torch.equal(am.view(T, E), aff) and torch.equal(tp, ltp)
        assert torch.equal(b2e, lb2e) and torch.equal(cond, lcond)
        arrays.update({f"c{i}_aff": aff.numpy(), f"c{i}_aff_masked": am.view(-1).numpy(),
                       f"c{i}_tp2id": tp.numpy(), f"c{i}_b2e": b2e.numpy(),
                       f"c{i}_conditions": cond.numpy(),
                       f"c{i}_shape": np.array([T, E, K, B], dtype=np.int64)})
    np.savez(HERE / "blockwise.npz", **arrays)


def router_case():
    T, E, H, K = 9, 16, 64, 4
    x = synthetic.normal_bf16(901, (T, H), 1.0)
    w = synthetic.normal_bf16(902, (E, H), 0.05)
    aff, logits = orr.router(x, w.T, K, return_logits=True)
    ld = x.double() @ w.double().T
    srt = torch.sort(ld, 1, descending=True)
    gap = (srt.values[:, K - 1] - srt.values[:, K]).min().item()
    assert gap > 1e-3, gap  # tie-free: fp32 summation order cannot swap the selection
    ids = srt.indices[:, :K]
    want = torch.softmax(srt.values[:, :K], 1)
    got_ids = torch.topk(aff, K, dim=1).indices
    assert torch.equal(torch.sort(got_ids, 1).values, torch.sort(ids, 1).values)
    assert torch.allclose(aff.gather(1, ids).double(), want, rtol=1e-6, atol=1e-7)
    np.savez(HERE / "router.npz", x_bits=x.view(torch.int16).numpy(),
             w_bits=w.view(torch.int16).numpy(), logits=logits.numpy(), topk_ids=ids.numpy(),
             topk_vals=want.float().numpy(), affinities=aff.numpy(),
             shape=np.array([T, E, H, K], dtype=np.int64))


def tiny_layer():
    shape = synthetic.MoEShape("tiny", 4, 2, 64, 64)
    lt = synthetic.layer_tensors(shape, 11, exp_range=(118, 122))
    ref = RefLayer(lt)
    x = synthetic.tokens(12, 5, 64)
    dec, aff_d = ref.decode(x)
    pre, aff_p = ref.prefill(x)
    assert torch.equal(aff_d, aff_p)
    # float64 closed form of the routed expert MLP (no bf16 roundings): the fp32
    # decode flow must sit within float32 accumulation error of it.
    gu = ref.gate_up.double().reshape(4, 64, 2, 64)
    dn = ref.down.double()
    gb = ref.gu_bias.double().reshape(4, 2, 64)
    out = torch.zeros(5, 64, dtype=torch.float64)
    xd = x.double()
    for t in range(5):
        for e in torch.nonzero(aff_d[t]).flatten().tolist():
            g = xd[t] @ gu[e, :, 0] + gb[e, 0]
            u = xd[t] @ gu[e, :, 1] + gb[e, 1]
            g = torch.clamp(g, max=7.0)
            u = torch.clamp(u, -6.0, 8.0)
            h = u * g * torch.sigmoid(1.702 * g)
            out[t] += aff_d[t, e].double() * (h @ dn[e] + ref.dn_bias[e].double())
    rel = ((dec.double() - out).abs().max() / out.abs().max()).item()
    assert rel < 1e-2, rel  # bf16 output rounding dominates
    np.savez(HERE / "tiny_layer.npz",
             x_bits=x.view(torch.int16).numpy(),
             gate_up_blocks=lt.gate_up_blocks.numpy(), gate_up_scales=lt.gate_up_scales.numpy(),
             down_blocks=lt.down_blocks.numpy(), down_scales=lt.down_scales.numpy(),
             gate_up_bias_bits=lt.gate_up_bias.view(torch.int16).numpy(),
             down_bias_bits=lt.down_bias.view(torch.int16).numpy(),
             router_w_bits=lt.router_w.view(torch.int16).numpy(),
             affinities=aff_d.numpy(), decode_bits=dec.view(torch.int16).numpy(),
             prefill_f32=pre.float().numpy(),
             shape=np.array([4, 2, 64, 64, 5], dtype=np.int64))


SHA_SHAPES = {  # name -> (shape, seed, E override, zipf)
    "gptoss20b_seed1": (synthetic.GPT_OSS_20B, 1, None, None),
    "mini_E8_seed3": (synthetic.MoEShape("mini", 8, 2, 256, 512), 3, None, None),
}


def synthetic_hashes():
    out = {}
    for name, (shape, seed, E, zipf) in SHA_SHAPES.items():
        lt = synthetic.layer_tensors(shape, seed, zipf_s=zipf, E=E)
        out[name] = {f: synthetic.sha256(getattr(lt, f)) for f in
                     ("gate_up_blocks", "gate_up_scales", "down_blocks", "down_scales",
                      "gate_up_bias", "down_bias", "router_w")}
    out["tokens_seed21_T64_H2880"] = synthetic.sha256(synthetic.tokens(21, 64, 2880))
    (HERE / "synthetic_sha256.json").write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")


if __name__ == "__main__":
    dequant_kat()
    packed_layout()
    blockwise()
    router_case()
    tiny_layer()
    synthetic_hashes()
    print("golden fixtures written to", HERE)
