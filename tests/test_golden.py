"""The committed golden fixtures (tests/golden/, written by make_golden.py) against the
oracle and the product's host-side packing, on the CPU."""

import json
from pathlib import Path

import numpy as np
import torch

from moe_helpers import MAX_REL, MEAN_REL
from oracle import blockwise as ob
from oracle import mxfp4 as om
from oracle import router as orr

G = Path(__file__).resolve().parent / "golden"


def load(name):
    return np.load(G / name)  # allow_pickle=False by default


def test_dequant_kat():
    d = load("dequant_kat.npz")
    assert np.array_equal(d["fp4_lut"], np.array(om.FP4_VALUES, dtype=np.float32))
    out = om.dequantize_mxfp4_to_bf16(torch.from_numpy(d["blocks"]), torch.from_numpy(d["scales"]))
    bits = out.view(torch.int16).numpy().astype(np.uint16).reshape(256, 32)
    assert np.array_equal(bits, d["bf16_bits"])


def test_packed_layout():
    from vllm_neuron_amd.weights import pack_mxfp4, unpack_mxfp4

    d = load("packed_layout.npz")
    pd, ps = pack_mxfp4(torch.from_numpy(d["blocks"]), torch.from_numpy(d["scales"]))
    assert np.array_equal(pd.numpy(), d["packed_data"])
    assert np.array_equal(ps.numpy(), d["packed_scales"])
    b, s = unpack_mxfp4(pd, ps)
    assert np.array_equal(b.numpy(), d["blocks"]) and np.array_equal(s.numpy(), d["scales"])


def test_blockwise_cases():
    d = load("blockwise.npz")
    i = 0
    while f"c{i}_shape" in d:
        T, E, K, B = (int(v) for v in d[f"c{i}_shape"])
        aff = torch.from_numpy(d[f"c{i}_aff"])
        am, tp, b2e, cond = ob.build_blockwise_mapping(aff, E, K, B)
        assert np.array_equal(am.view(-1).numpy(), d[f"c{i}_aff_masked"])
        assert np.array_equal(tp.numpy(), d[f"c{i}_tp2id"])
        assert np.array_equal(b2e.numpy(), d[f"c{i}_b2e"])
        assert np.array_equal(cond.numpy(), d[f"c{i}_conditions"])
        assert len(tp) == ob.num_blocks(T, E, K, B) * B
        i += 1
    assert i == 5


def test_router_case():
    d = load("router.npz")
    T, E, H, K = (int(v) for v in d["shape"])
    x = torch.from_numpy(d["x_bits"]).view(torch.bfloat16)
    w = torch.from_numpy(d["w_bits"]).view(torch.bfloat16)
    aff, logits = orr.router(x, w.T, K, return_logits=True)
    assert torch.allclose(logits, torch.from_numpy(d["logits"]), rtol=1e-6, atol=1e-6)
    ids = torch.from_numpy(d["topk_ids"])
    assert torch.equal(torch.sort(torch.topk(aff, K, 1).indices, 1).values,
                       torch.sort(ids, 1).values)
    assert torch.allclose(aff.gather(1, ids), torch.from_numpy(d["topk_vals"]), rtol=1e-6,
                          atol=1e-7)


def tiny_layer_tensors(d):
    from vllm_neuron_amd import synthetic

    t = lambda k: torch.from_numpy(d[k])  # noqa: E731
    shape = synthetic.MoEShape("tiny", 4, 2, 64, 64)
    lt = synthetic.LayerTensors(shape, t("gate_up_blocks"), t("gate_up_scales"),
                                t("down_blocks"), t("down_scales"),
                                t("gate_up_bias_bits").view(torch.bfloat16),
                                t("down_bias_bits").view(torch.bfloat16),
                                t("router_w_bits").view(torch.bfloat16), None)
    return lt, t("x_bits").view(torch.bfloat16)


def rel_errors(got, want):
    d = (got.double() - want.double()).abs()
    return (d.max() / want.double().abs().max()).item(), (d.mean() / want.double().abs().mean()).item()


def test_tiny_layer_oracle():
    from oracle.layer import RefLayer

    d = load("tiny_layer.npz")
    lt, x = tiny_layer_tensors(d)
    ref = RefLayer(lt)
    dec, aff = ref.decode(x)
    assert torch.equal(aff, torch.from_numpy(d["affinities"]))
    mx, mean = rel_errors(dec, torch.from_numpy(d["decode_bits"]).view(torch.bfloat16))
    assert mx <= 1e-2 and mean <= 1e-3, (mx, mean)  # float summation order only
    pre, _ = ref.prefill(x)
    mx, mean = rel_errors(pre, torch.from_numpy(d["prefill_f32"]))
    assert mx <= MAX_REL and mean <= MEAN_REL, (mx, mean)


def test_synthetic_generator_hashes():
    import sys

    sys.path.insert(0, str(G))
    from make_golden import SHA_SHAPES

    from vllm_neuron_amd import synthetic

    want = json.loads((G / "synthetic_sha256.json").read_text())
    name = "mini_E8_seed3"  # the small shape: the 20B one takes long on one core
    shape, seed, E, zipf = SHA_SHAPES[name]
    lt = synthetic.layer_tensors(shape, seed, zipf_s=zipf, E=E)
    for f, h in want[name].items():
        assert synthetic.sha256(getattr(lt, f)) == h, f
    assert synthetic.sha256(synthetic.tokens(21, 64, 2880)) == want["tokens_seed21_T64_H2880"]
