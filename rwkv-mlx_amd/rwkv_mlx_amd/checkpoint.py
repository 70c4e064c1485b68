"""Checkpoint I/O for the MoE ChannelMix layers under the reference's
parameter names, so MLX checkpoints load into the torch drop-in and the
delta files it writes load back into MLX.

Names (rwkv_mlx/moe.py:47, 113, 124-127, 190-209; model.py:253-257), for
block i.  LoRA experts (LoRAMoE_CMix):

    blocks.{i}.ffn.base.x_k            (1, 1, C)
    blocks.{i}.ffn.base.key.weight     (F, C)
    blocks.{i}.ffn.base.value.weight   (C, F)
    blocks.{i}.ffn.lora_A              (E, C, r)
    blocks.{i}.ffn.lora_B              (E, r, C)
    blocks.{i}.ffn.router.gate.weight  (E, C)

full experts (MoE_CMix):

    blocks.{i}.ffn.x_k                 (E, 1, 1, C)
    blocks.{i}.ffn.expert_key          (E, F, C)
    blocks.{i}.ffn.expert_val          (E, C, F)
    blocks.{i}.ffn.router.gate.weight  (E, C)

A dense (non-MoE) checkpoint holds the base ChannelMix as
``blocks.{i}.ffn.{x_k,key.weight,value.weight}``; ``build_moe_from_base``
injects those into a fresh MoE layer the way rwkv_mlx/finetune_moe.py:47-86
does (the ``.ffn.base.`` -> ``.ffn.`` name translation; every other tensor
keeps its fresh initialisation).  ``save_expert_weights`` writes the tensors
finetune_moe.py:89-109 selects: names holding ``.ffn.lora_A``,
``.ffn.lora_B``, ``.ffn.router.`` or ``.ffn.x_k`` — the adapters and router
of a LoRA layer, the router and the per-expert x_k of a full layer (whose
expert_key / expert_val that filter leaves out).

Files are read with safetensors only (no pickle); tensors keep the dtype the
file stores, as MLX ``load_weights`` does.
"""
from __future__ import annotations

from pathlib import Path

import torch

from .moe import LoRAMoE_CMix, MoE_CMix, RWKVConfig, build_layer

# module attribute path -> name under "blocks.{i}.ffn."
MOE_NAMES = {
    "base.x_k": "base.x_k",
    "base.key.weight": "base.key.weight",
    "base.value.weight": "base.value.weight",
    "lora_A": "lora_A",
    "lora_B": "lora_B",
    "router.gate.weight": "router.gate.weight",
}
# module attribute path -> name under "blocks.{i}.ffn." for a full-expert layer
FULL_NAMES = {
    "x_k": "x_k",
    "expert_key": "expert_key",
    "expert_val": "expert_val",
    "router.gate.weight": "router.gate.weight",
}
# the delta file's tensors (finetune_moe.py:98-106: the names holding .ffn.lora_A,
# .ffn.lora_B, .ffn.router. or .ffn.x_k)
EXPERT_NAMES = ("lora_A", "lora_B", "router.gate.weight")
FULL_EXPERT_NAMES = ("router.gate.weight", "x_k")


def layer_names(layer) -> dict[str, str]:
    """Attribute path -> checkpoint name (under ``blocks.{i}.ffn.``) of every
    tensor of a LoRAMoE_CMix or MoE_CMix."""
    if isinstance(layer, MoE_CMix):
        return FULL_NAMES
    if isinstance(layer, LoRAMoE_CMix):
        return MOE_NAMES
    raise TypeError(f"not an MoE ChannelMix layer: {type(layer).__name__}")


def delta_names(layer) -> tuple[str, ...]:
    """The tensors save_expert_weights writes for this layer."""
    return FULL_EXPERT_NAMES if isinstance(layer, MoE_CMix) else EXPERT_NAMES


def prefix(layer_id: int) -> str:
    return f"blocks.{layer_id}.ffn."


def load_safetensors(path: str | Path) -> dict[str, torch.Tensor]:
    """All tensors of a .safetensors file, on the CPU."""
    from safetensors.torch import load_file
    return load_file(str(path), device="cpu")


def _param(layer, path: str) -> torch.nn.Parameter:
    obj = layer
    for part in path.split("."):
        obj = getattr(obj, part)
    return obj


def _assign(layer, path: str, value: torch.Tensor, key: str) -> None:
    p = _param(layer, path)
    if tuple(value.shape) != tuple(p.shape):
        raise ValueError(f"{key}: checkpoint shape {tuple(value.shape)} != parameter shape {tuple(p.shape)}")
    p.data = value.detach().to(device=p.device).clone()
    # the layer's cached kernel layouts (LoRAMoE_CMix) are remade from the new values
    if hasattr(layer, "invalidate_prepared"):
        layer.invalidate_prepared()


def load_moe_layer(layer, tensors: dict[str, torch.Tensor], layer_id: int, strict: bool = True) -> list[str]:
    """Copy block ``layer_id``'s MoE ChannelMix tensors into ``layer`` (a
    LoRAMoE_CMix or an MoE_CMix).

    strict: every tensor of the layer must be present.  Returns the names
    that were loaded.  Shapes must match the layer's; the dtype is the
    file's."""
    pre = prefix(layer_id)
    loaded, missing = [], []
    for path, name in layer_names(layer).items():
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
                        top_k: int = 2, mode: str = "lora"):
    """A fresh MoE layer built from a dense checkpoint's base ChannelMix
    (``blocks.{i}.ffn.x_k / key.weight / value.weight``) or an MoE one
    (``blocks.{i}.ffn.base.*``).

    mode "lora" (LoRAMoE_CMix): the base takes those tensors; lora_A ~
    N(0,1)·0.01, lora_B = 0 and the router gate keep their initialisation,
    so the layer's delta starts at 0.

    mode "full" (MoE_CMix, lora_rank unused): of the layer's names only
    ``ffn.x_k`` has a dense counterpart, so only x_k is taken from the file;
    expert_key (orthogonal), expert_val (zeros) and the router keep their
    initialisation.  The dense x_k is (1, 1, C) against the layer's
    (E, 1, 1, C): every expert gets it (finetune_moe.py:66-84 assigns the
    (1, 1, C) array as it is, whose x_k[0] is the same vector).  An
    ``ffn.x_k`` already of shape (E, 1, 1, C) is taken as it is."""
    pre = prefix(layer_id)
    if mode == "full":
        key = pre + "x_k"
        if key not in tensors:
            raise KeyError(f"no ChannelMix tensor {key} in the checkpoint")
        xk = tensors[key]
        kw = pre + "expert_key"
        if kw in tensors:
            F, C = tensors[kw].shape[1:]
        else:
            for cand in (pre + "key.weight", pre + "base.key.weight"):
                if cand in tensors:
                    F, C = tensors[cand].shape
                    break
            else:
                raise KeyError(f"no {pre}key.weight or {pre}expert_key in the checkpoint to size the experts")
        layer = MoE_CMix(RWKVConfig(n_embd=C, dim_ffn=F), layer_id, n_experts, top_k)
        if xk.dim() == 3 and tuple(xk.shape) == (1, 1, C):
            xk = xk.reshape(1, 1, 1, C).expand(n_experts, 1, 1, C).contiguous()
        _assign(layer, "x_k", xk, key)
        return layer
    if mode != "lora":
        raise ValueError(f"mode must be 'lora' or 'full', got {mode!r}")
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


def expert_state(layers: dict) -> dict[str, torch.Tensor]:
    """The tensors of each block that save_expert_weights writes, under
    checkpoint names: adapters and router of a LoRA layer, router and x_k of
    a full layer."""
    out = {}
    for i, layer in layers.items():
        for name in delta_names(layer):
            out[prefix(i) + name] = _param(layer, name).detach().to("cpu").contiguous()
    return out


def moe_state(layers: dict) -> dict[str, torch.Tensor]:
    """Every MoE ChannelMix tensor of each block, under checkpoint names."""
    out = {}
    for i, layer in layers.items():
        for path, name in layer_names(layer).items():
            out[prefix(i) + name] = _param(layer, path).detach().to("cpu").contiguous()
    return out


def save_expert_weights(layers: dict, path: str | Path) -> None:
    """Write the delta file (finetune_moe.py:89-109) of the given blocks."""
    from safetensors.torch import save_file
    save_file(expert_state(layers), str(path))


def save_moe_weights(layers: dict, path: str | Path) -> None:
    """Write every MoE ChannelMix tensor of the given blocks."""
    from safetensors.torch import save_file
    save_file(moe_state(layers), str(path))
