"""Loading a GPT-OSS MoE layer from a (synthetic) safetensors checkpoint (CPU)."""

import json

import pytest
import torch


def _write_checkpoint(tmp_path, sharded):
    from safetensors.torch import save_file

    from vllm_neuron_amd import synthetic

    shape = synthetic.MoEShape("ck", 4, 2, 64, 96)
    lt = synthetic.layer_tensors(shape, 61)
    gamma = torch.linspace(0.5, 1.5, 64)
    tensors = {
        "model.layers.3.mlp.router.weight": lt.router_w,
        "model.layers.3.mlp.router.bias": torch.zeros(4, dtype=torch.bfloat16),
        "model.layers.3.mlp.experts.gate_up_proj_blocks": lt.gate_up_blocks,
        "model.layers.3.mlp.experts.gate_up_proj_scales": lt.gate_up_scales,
        "model.layers.3.mlp.experts.gate_up_proj_bias": lt.gate_up_bias,
        "model.layers.3.mlp.experts.down_proj_blocks": lt.down_blocks,
        "model.layers.3.mlp.experts.down_proj_scales": lt.down_scales,
        "model.layers.3.mlp.experts.down_proj_bias": lt.down_bias,
        "model.layers.3.post_attention_layernorm.weight": gamma,
        "model.layers.3.self_attn.o_proj.weight": torch.zeros(8, 8),
    }
    if not sharded:
        save_file(tensors, str(tmp_path / "model.safetensors"))
    else:
        names = sorted(tensors)
        a, b = names[: len(names) // 2], names[len(names) // 2:]
        save_file({k: tensors[k] for k in a}, str(tmp_path / "model-00001-of-00002.safetensors"))
        save_file({k: tensors[k] for k in b}, str(tmp_path / "model-00002-of-00002.safetensors"))
        wm = {k: "model-00001-of-00002.safetensors" for k in a}
        wm.update({k: "model-00002-of-00002.safetensors" for k in b})
        (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    return lt, gamma


@pytest.mark.parametrize("sharded", [False, True])
def test_load_moe_layer(tmp_path, sharded):
    from vllm_neuron_amd.checkpoint import load_moe_layer
    from vllm_neuron_amd.weights import MXFP4Experts

    lt, gamma = _write_checkpoint(tmp_path, sharded)
    w = load_moe_layer(tmp_path, 3)
    want = MXFP4Experts.from_checkpoint(lt.gate_up_blocks, lt.gate_up_scales, lt.down_blocks,
                                        lt.down_scales, lt.gate_up_bias, lt.down_bias)
    for name in ("gu_q", "gu_s", "dn_q", "dn_s", "gu_bias", "dn_bias"):
        assert torch.equal(getattr(w.experts, name), getattr(want, name)), name
    assert (w.experts.E, w.experts.H, w.experts.I) == (4, 64, 96)
    assert torch.equal(w.router_w, lt.router_w)
    assert torch.equal(w.norm_gamma, gamma)


def test_load_errors(tmp_path):
    from vllm_neuron_amd.checkpoint import load_moe_layer

    _write_checkpoint(tmp_path, False)
    with pytest.raises(KeyError):
        load_moe_layer(tmp_path, 0)
    (tmp_path / "empty").mkdir()
    with pytest.raises(FileNotFoundError):
        load_moe_layer(tmp_path / "empty", 3)
