"""Checkpoint I/O for the MoE ChannelMix layers under the reference's
parameter names, so MLX checkpoints load into the torch drop-in and the
delta files it writes load back into MLX.

Names (rwkv_mlx/moe.py:47, 113, 124-127; model.py:253-257), for block i:

    blocks.{i}.ffn.base.x_k            (1, 1, C)
    blocks.{i}.ffn.base.key.weight     (F, C)
    blocks.{i}.ffn.base.value.weight   (C, F)
    blocks.{i}.ffn.lora_A              (E, C, r)
    blocks.{i}.ffn.lora_B              (E, r, C)
    blocks.{i}.ffn.router.gate.weight  (E, C)

A dense (non-MoE) checkpoint holds the base ChannelMix as
``blocks.{i}.ffn.{x_k,key.weight,value.weight}``; ``build_moe_from_base``
injects those into a fresh MoE layer the way rwkv_mlx/finetune_moe.py:47-86
does (the ``.ffn.base.`` -> ``.ffn.`` name translation; adapters and router
keep their fresh initialisation).  ``save_expert_weights`` writes only the
adapter and router tensors (finetune_moe.py:89-109).

Files are read with safetensors only (no pickle); tensors keep the dtype the
file stores, as MLX ``load_weights`` does.
"""
from __future__ import annotations

from pathlib import Path

import torch

from .moe import LoRAMoE_CMix, build_layer

# module attribute path -> name under "blocks.{i}.ffn."
MOE_NAMES = {
    "base.x_k": "base.x_k",
    "base.key.weight": "base.key.weight",
    "base.value.weight": "base.value.weight",
    "lora_A": "lora_A",
    "lora_B": "lora_B",
    "router.gate.weight": "router.gate.weight",
}
# the delta file's tensors (finetune_moe.py:98-104)
EXPERT_NAMES = ("lora_A", "lora_B", "router.gate.weight")


def prefix(layer_id: int) -> str:
    return f"blocks.{layer_id}.ffn."


def load_safetensors(path: str | Path) -> dict[str, torch.Tensor]:
    """All tensors of a .safetensors file, on the CPU."""
    from safetensors.torch import load_file
    return load_file(str(path), device="cpu")


def _param(layer: LoRAMoE_CMix, path: str) -> torch.nn.Parameter:
    obj = layer
    for part in path.split("."):
        obj = getattr(obj, part)
    return obj


def _assign(layer: LoRAMoE_CMix, path: str, value: torch.Tensor, key: str) -> None:
    p = _param(layer, path)
    if tuple(value.shape) != tuple(p.shape):
        raise ValueError(f"{key}: checkpoint shape {tuple(value.shape)} != parameter shape {tuple(p.shape)}")
    p.data = value.detach().to(device=p.device).clone()


def load_moe_layer(layer: LoRAMoE_CMix, tensors: dict[str, torch.Tensor], layer_id: int,
                   strict: bool = True) -> list[str]:
    """Copy block ``layer_id``'s MoE ChannelMix tensors into ``layer``.

    strict: every one of the six tensors must be present.  Returns the
    names that were loaded.  Shapes must match the layer's; the dtype is the
    file's."""
    pre = prefix(layer_id)
    loaded, missing = [], []
    for path, name in MOE_NAMES.items():
        key = pre + name
        if key in tensors:
            _assign(layer, path, tensors[key], key)
            loaded.append(key)
        else:
            missing.append(key)
    if strict and missing:
        raise KeyError(f"missing from the checkpoint: {', '.join(missing)}")
    return loaded


def build_moe_from_base(tensors: dict[str, torch.Tensor], layer_id: int, n_experts: int, lora_rank: int,
                        top_k: int = 2) -> LoRAMoE_CMix:
    """A fresh MoE layer whose base ChannelMix comes from a dense checkpoint
    (``blocks.{i}.ffn.x_k / key.weight / value.weight``) or an MoE one
    (``blocks.{i}.ffn.base.*``); lora_A ~ N(0,1)·0.01, lora_B = 0 and the
    router gate keep their initialisation, so the layer's delta starts at 0."""
    pre = prefix(layer_id)
    found = {}
    for path in ("x_k", "key.weight", "value.weight"):
        for key in (pre + "base." + path, pre + path):
            if key in tensors:
                found[path] = (key, tensors[key])
                break
        else:
            raise KeyError(f"no base ChannelMix tensor {pre}{path} (or {pre}base.{path}) in the checkpoint")
    F, C = found["key.weight"][1].shape
    layer = build_layer(C, F, n_experts, top_k, lora_rank)
    for path, (key, t) in found.items():
        _assign(layer, "base." + path, t, key)
    return layer


def expert_state(layers: dict[int, LoRAMoE_CMix]) -> dict[str, torch.Tensor]:
    """The adapter and router tensors of each block, under checkpoint names."""
    out = {}
    for i, layer in layers.items():
        for name in EXPERT_NAMES:
            out[prefix(i) + name] = _param(layer, name).detach().to("cpu").contiguous()
    return out


def moe_state(layers: dict[int, LoRAMoE_CMix]) -> dict[str, torch.Tensor]:
    """Every MoE ChannelMix tensor of each block, under checkpoint names."""
    out = {}
    for i, layer in layers.items():
        for path, name in MOE_NAMES.items():
            out[prefix(i) + name] = _param(layer, path).detach().to("cpu").contiguous()
    return out


def save_expert_weights(layers: dict[int, LoRAMoE_CMix], path: str | Path) -> None:
    """Write the delta-only file (lora_A, lora_B, router.gate.weight per block)."""
    from safetensors.torch import save_file
    save_file(expert_state(layers), str(path))


def save_moe_weights(layers: dict[int, LoRAMoE_CMix], path: str | Path) -> None:
    """Write every MoE ChannelMix tensor of the given blocks."""
    from safetensors.torch import save_file
    save_file(moe_state(layers), str(path))
