"""GPT-OSS MoE layer weights from a Hugging Face safetensors checkpoint.

The reference maps these checkpoint keys onto its MoE parameters
(vllm_neuron/model/gpt_oss/model_mxfp4.py:2069-2141):

  model.layers.{i}.mlp.router.weight / .bias                 router [E, H], [E]
  model.layers.{i}.mlp.experts.gate_up_proj_blocks / _scales [E, 2I, H/32, 16], [E, 2I, H/32]
  model.layers.{i}.mlp.experts.gate_up_proj_bias             [E, 2I] (gate/up rows interleaved)
  model.layers.{i}.mlp.experts.down_proj_blocks / _scales    [E, H, I/32, 16], [E, H, I/32]
  model.layers.{i}.mlp.experts.down_proj_bias                [E, H]
  model.layers.{i}.post_attention_layernorm.weight           the RMSNorm gamma before the MoE

``load_moe_layer`` reads one layer (only its tensors, through safetensors' lazy
access) and returns packed experts, the router and the norm gamma; ``moe_layer``
builds the layer object on a device.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, Optional, Union

import torch

from .weights import MXFP4Experts

PathLike = Union[str, Path]

_EXPERT_KEYS = ("gate_up_proj_blocks", "gate_up_proj_scales", "gate_up_proj_bias",
                "down_proj_blocks", "down_proj_scales", "down_proj_bias")


def _key_to_file(path: Path) -> Dict[str, Path]:
    """Tensor name -> shard file, from model.safetensors.index.json when present."""
    if path.is_file():
        from safetensors import safe_open

        with safe_open(str(path), framework="pt") as f:
            return {k: path for k in f.keys()}
    index = path / "model.safetensors.index.json"
    if index.exists():
        weight_map = json.loads(index.read_text())["weight_map"]
        return {k: path / v for k, v in weight_map.items()}
    from safetensors import safe_open

    out = {}
    for shard in sorted(path.glob("*.safetensors")):
        with safe_open(str(shard), framework="pt") as f:
            out.update({k: shard for k in f.keys()})
    if not out:
        raise FileNotFoundError(f"no safetensors files under {path}")
    return out


def _read(files: Dict[str, Path], key: str, required: bool = True) -> Optional[torch.Tensor]:
    from safetensors import safe_open

    if key not in files:
        if required:
            raise KeyError(f"checkpoint has no tensor {key}")
        return None
    with safe_open(str(files[key]), framework="pt") as f:
        return f.get_tensor(key)


@dataclass
class MoELayerWeights:
    experts: MXFP4Experts
    router_w: torch.Tensor            # [E, H] bf16
    router_b: Optional[torch.Tensor]  # [E] bf16
    norm_gamma: Optional[torch.Tensor]  # [H]


def load_moe_layer(checkpoint: PathLike, layer: int, up_bias_offset: float = 1.0) -> MoELayerWeights:
    """Expert, router and norm tensors of one layer, packed for the kernels (CPU)."""
    files = _key_to_file(Path(checkpoint))
    p = f"model.layers.{layer}"
    t = {k: _read(files, f"{p}.mlp.experts.{k}", required=not k.endswith("bias"))
         for k in _EXPERT_KEYS}
    for k in ("gate_up_proj_blocks", "gate_up_proj_scales", "down_proj_blocks",
              "down_proj_scales"):
        if t[k].dtype != torch.uint8:
            raise TypeError(f"{p}.mlp.experts.{k}: expected uint8 MXFP4 data, got {t[k].dtype}")
    experts = MXFP4Experts.from_checkpoint(t["gate_up_proj_blocks"], t["gate_up_proj_scales"],
                                           t["down_proj_blocks"], t["down_proj_scales"],
                                           t["gate_up_proj_bias"], t["down_proj_bias"],
                                           up_bias_offset=up_bias_offset)
    router_w = _read(files, f"{p}.mlp.router.weight")
    if tuple(router_w.shape) != (experts.E, experts.H):
        raise ValueError(f"router weight shape {tuple(router_w.shape)} does not match "
                         f"E={experts.E}, H={experts.H}")
    return MoELayerWeights(experts, router_w.to(torch.bfloat16),
                           _read(files, f"{p}.mlp.router.bias", required=False),
                           _read(files, f"{p}.post_attention_layernorm.weight", required=False))


def moe_layer(checkpoint: PathLike, layer: int, device, top_k: int = 4,
              swiglu_limit: Optional[float] = 7.0):
    """The MXFP4MoE layer object of one checkpoint layer on ``device`` (GPT-OSS: top-4,
    clamped SwiGLU with limit 7)."""
    from .layer import MXFP4MoE

    w = load_moe_layer(checkpoint, layer)
    rb = None if w.router_b is None else w.router_b.to(device=device, dtype=torch.bfloat16)
    return MXFP4MoE(w.experts.to(device), w.router_w.to(device), rb, top_k, swiglu_limit)
