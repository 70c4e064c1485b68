"""Checkpoint I/O under the reference's parameter names
(rwkv_mlx/moe.py:47, 113, 124-127; model.py:253-257; finetune_moe.py:47-109):
an MoE checkpoint loads into the torch drop-in with the file's values and
dtypes; a dense checkpoint's base ChannelMix is injected with fresh adapters
(zero delta); the delta file holds exactly the adapter and router tensors (router and
x_k for a full-expert layer);
save -> load round trips are exact.  The last test runs a loaded layer on the
GPU and checks it against the same layer built in memory."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from rwkv_mlx_amd import checkpoint as ck
from rwkv_mlx_amd.moe import build_layer

C, F, E, R, K = 64, 128, 4, 8, 2


def _moe_file(tmp_path, layer_ids=(0, 3), dtype=torch.bfloat16, seed=0):
    """A checkpoint laid out as MLX's save_safetensors writes an MoE model's
    tree_flatten(parameters()) (plus a non-FFN tensor that must be ignored)."""
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(seed)
    t = {"emb.weight": torch.randn(10, C, generator=g).to(dtype)}
    for i in layer_ids:
        p = ck.prefix(i)
        t[p + "base.x_k"] = torch.rand(1, 1, C, generator=g).to(dtype)
        t[p + "base.key.weight"] = torch.randn(F, C, generator=g).to(dtype)
        t[p + "base.value.weight"] = torch.randn(C, F, generator=g).to(dtype)
        t[p + "lora_A"] = torch.randn(E, C, R, generator=g).to(dtype)
        t[p + "lora_B"] = torch.randn(E, R, C, generator=g).to(dtype)
        t[p + "router.gate.weight"] = torch.randn(E, C, generator=g).to(dtype)
    path = tmp_path / "moe.safetensors"
    save_file(t, str(path))
    return path, t


def test_load_moe_checkpoint_values_and_dtypes(tmp_path):
    path, ref = _moe_file(tmp_path)
    tensors = ck.load_safetensors(path)
    layer = build_layer(C, F, E, K, R)
    loaded = ck.load_moe_layer(layer, tensors, 3)
    assert sorted(loaded) == sorted(ck.prefix(3) + n for n in ck.MOE_NAMES.values())
    for path_, name in ck.MOE_NAMES.items():
        p = ck._param(layer, path_)
        want = ref[ck.prefix(3) + name]
        assert p.dtype == want.dtype == torch.bfloat16
        assert torch.equal(p.detach(), want)


def test_missing_and_mismatched_tensors_raise(tmp_path):
    path, ref = _moe_file(tmp_path, layer_ids=(0,))
    tensors = ck.load_safetensors(path)
    layer = build_layer(C, F, E, K, R)
    with pytest.raises(KeyError):
        ck.load_moe_layer(layer, tensors, 1)  # block 1 is not in the file
    assert ck.load_moe_layer(layer, tensors, 1, strict=False) == []
    wrong = build_layer(C, F, E, K, R * 2)  # rank 16 against a rank-8 file
    with pytest.raises(ValueError, match="lora_A"):
        ck.load_moe_layer(wrong, tensors, 0)


def test_build_moe_from_dense_base(tmp_path):
    """finetune_moe.py:47-86: blocks.i.ffn.{x_k,key,value} -> ffn.base.*, the
    adapters keep their initialisation (lora_B = 0, so the delta is zero)."""
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(1)
    t = {"blocks.2.ffn.x_k": torch.rand(1, 1, C, generator=g),
         "blocks.2.ffn.key.weight": torch.randn(F, C, generator=g),
         "blocks.2.ffn.value.weight": torch.randn(C, F, generator=g),
         "blocks.2.att.r_k": torch.randn(4, 16, generator=g)}
    save_file(t, str(tmp_path / "base.safetensors"))
    tensors = ck.load_safetensors(tmp_path / "base.safetensors")
    layer = ck.build_moe_from_base(tensors, 2, n_experts=E, lora_rank=R, top_k=K)
    assert torch.equal(layer.base.x_k.detach(), t["blocks.2.ffn.x_k"])
    assert torch.equal(layer.base.key.weight.detach(), t["blocks.2.ffn.key.weight"])
    assert torch.equal(layer.base.value.weight.detach(), t["blocks.2.ffn.value.weight"])
    assert tuple(layer.lora_A.shape) == (E, C, R) and tuple(layer.lora_B.shape) == (E, R, C)
    assert torch.count_nonzero(layer.lora_B) == 0
    assert (layer.n_experts, layer.top_k, layer.lora_rank) == (E, K, R)
    with pytest.raises(KeyError):
        ck.build_moe_from_base(tensors, 0, E, R, K)


def test_expert_delta_file_and_round_trip(tmp_path):
    path, ref = _moe_file(tmp_path, dtype=torch.float32)
    tensors = ck.load_safetensors(path)
    layers = {}
    for i in (0, 3):
        layers[i] = build_layer(C, F, E, K, R)
        ck.load_moe_layer(layers[i], tensors, i)
    ck.save_expert_weights(layers, tmp_path / "delta.safetensors")
    delta = ck.load_safetensors(tmp_path / "delta.safetensors")
    assert sorted(delta) == sorted(ck.prefix(i) + n for i in (0, 3) for n in ck.EXPERT_NAMES)
    for key, v in delta.items():
        assert torch.equal(v, ref[key])
    ck.save_moe_weights(layers, tmp_path / "full.safetensors")
    full = ck.load_safetensors(tmp_path / "full.safetensors")
    again = build_layer(C, F, E, K, R)
    ck.load_moe_layer(again, full, 3)
    for path_ in ck.MOE_NAMES:
        assert torch.equal(ck._param(again, path_).detach(), ck._param(layers[3], path_).detach())
    # a delta file on top of a base-injected layer reproduces the full layer
    base_only = ck.build_moe_from_base(full, 3, E, R, K)
    ck.load_moe_layer(base_only, delta, 3, strict=False)
    for path_ in ck.MOE_NAMES:
        assert torch.equal(ck._param(base_only, path_).detach(), ck._param(layers[3], path_).detach())


def _full_file(tmp_path, layer_ids=(1,), dtype=torch.bfloat16, seed=2):
    """A full-expert (moe_mode "full") checkpoint as MLX writes MoE_CMix's
    parameters (moe.py:190-209)."""
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(seed)
    t = {"emb.weight": torch.randn(10, C, generator=g).to(dtype)}
    for i in layer_ids:
        p = ck.prefix(i)
        t[p + "x_k"] = torch.rand(E, 1, 1, C, generator=g).to(dtype)
        t[p + "expert_key"] = torch.randn(E, F, C, generator=g).to(dtype)
        t[p + "expert_val"] = torch.randn(E, C, F, generator=g).to(dtype)
        t[p + "router.gate.weight"] = torch.randn(E, C, generator=g).to(dtype)
    path = tmp_path / "full.safetensors"
    save_file(t, str(path))
    return path, t


def _full_layer():
    from rwkv_mlx_amd import MoE_CMix, RWKVConfig
    return MoE_CMix(RWKVConfig(n_embd=C, dim_ffn=F), 0, E, K)


def test_full_expert_checkpoint_load_delta_and_round_trip(tmp_path):
    """MoE_CMix's x_k / expert_key / expert_val / router.gate.weight load with
    the file's values and dtypes; the delta file holds what
    finetune_moe.py:98-106's name filter selects for a full layer (router and
    x_k); save -> load round trips are exact."""
    path, ref = _full_file(tmp_path)
    tensors = ck.load_safetensors(path)
    layer = _full_layer()
    loaded = ck.load_moe_layer(layer, tensors, 1)
    assert sorted(loaded) == sorted(ck.prefix(1) + n for n in ck.FULL_NAMES.values())
    for path_, name in ck.FULL_NAMES.items():
        p = ck._param(layer, path_)
        assert p.dtype == torch.bfloat16 and torch.equal(p.detach(), ref[ck.prefix(1) + name])
    with pytest.raises(KeyError):
        ck.load_moe_layer(_full_layer(), tensors, 0)
    ck.save_expert_weights({1: layer}, tmp_path / "delta.safetensors")
    delta = ck.load_safetensors(tmp_path / "delta.safetensors")
    assert sorted(delta) == [ck.prefix(1) + "router.gate.weight", ck.prefix(1) + "x_k"]
    ck.save_moe_weights({1: layer}, tmp_path / "all.safetensors")
    again = _full_layer()
    ck.load_moe_layer(again, ck.load_safetensors(tmp_path / "all.safetensors"), 1)
    for path_ in ck.FULL_NAMES:
        assert torch.equal(ck._param(again, path_).detach(), ck._param(layer, path_).detach())
    # a LoRA layer's and a full layer's names differ: loading one into the other fails
    with pytest.raises(KeyError):
        ck.load_moe_layer(build_layer(C, F, E, K, R), tensors, 1)


def test_build_full_moe_from_dense_base(tmp_path):
    """moe_mode "full" from a dense checkpoint: only ffn.x_k has a dense
    counterpart; every expert gets it, expert_key keeps its scaled
    orthogonal initialisation and expert_val its zeros."""
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(3)
    t = {"blocks.2.ffn.x_k": torch.rand(1, 1, C, generator=g),
         "blocks.2.ffn.key.weight": torch.randn(F, C, generator=g),
         "blocks.2.ffn.value.weight": torch.randn(C, F, generator=g)}
    save_file(t, str(tmp_path / "base.safetensors"))
    tensors = ck.load_safetensors(tmp_path / "base.safetensors")
    layer = ck.build_moe_from_base(tensors, 2, n_experts=E, lora_rank=R, top_k=K, mode="full")
    assert tuple(layer.x_k.shape) == (E, 1, 1, C)
    for e in range(E):
        assert torch.equal(layer.x_k[e].detach(), t["blocks.2.ffn.x_k"])
    assert torch.count_nonzero(layer.expert_val) == 0
    wk = layer.expert_key.detach()
    gram = wk[0].T @ wk[0]  # F >= C: orthonormal columns scaled by sqrt(F/C)
    assert torch.allclose(gram, torch.eye(C) * (F / C), atol=1e-4)
    with pytest.raises(KeyError):
        ck.build_moe_from_base(tensors, 0, E, R, K, mode="full")
    with pytest.raises(ValueError):
        ck.build_moe_from_base(tensors, 2, E, R, K, mode="dense")


@pytest.mark.gpu
def test_loaded_layer_runs_identically_on_gpu(tmp_path):
    path, ref = _moe_file(tmp_path, dtype=torch.float16)
    tensors = ck.load_safetensors(path)
    loaded = build_layer(C, F, E, K, R)
    ck.load_moe_layer(loaded, tensors, 0)
    direct = build_layer(C, F, E, K, R)
    with torch.no_grad():
        for path_, name in ck.MOE_NAMES.items():
            ck._param(direct, path_).data = ref[ck.prefix(0) + name].clone()
    loaded, direct = loaded.cuda(), direct.cuda()
    x = torch.randn(2, 16, C, generator=torch.Generator().manual_seed(5)).to(torch.float16).cuda()
    with torch.no_grad():
        a, la, za = loaded(x)
        b, lb, zb = direct(x)
    torch.cuda.synchronize()
    assert a.dtype == torch.float16
    assert np.array_equal(a.cpu().numpy(), b.cpu().numpy())
    assert float(la) == float(lb) and float(za) == float(zb)


@pytest.mark.gpu
def test_loaded_full_layer_runs_and_trains_on_gpu(tmp_path):
    """A full-expert layer loaded from a file runs as the same layer built in
    memory, and its backward reaches every loaded tensor."""
    path, ref = _full_file(tmp_path, layer_ids=(0,), dtype=torch.float16)
    tensors = ck.load_safetensors(path)
    loaded = _full_layer()
    ck.load_moe_layer(loaded, tensors, 0)
    direct = _full_layer()
    with torch.no_grad():
        for path_, name in ck.FULL_NAMES.items():
            ck._param(direct, path_).data = ref[ck.prefix(0) + name].clone()
    loaded, direct = loaded.cuda(), direct.cuda()
    x = torch.randn(2, 16, C, generator=torch.Generator().manual_seed(6)).to(torch.float16).cuda()
    with torch.no_grad():
        a, la, za = loaded(x)
        b, lb, zb = direct(x)
    torch.cuda.synchronize()
    assert np.array_equal(a.cpu().numpy(), b.cpu().numpy())
    assert float(la) == float(lb) and float(za) == float(zb)
    out, aux, z = loaded(x)
    (out.float().square().mean() + 0.01 * aux + 0.001 * z).backward()
    for path_ in ck.FULL_NAMES:
        gr = ck._param(loaded, path_).grad
        assert gr is not None and torch.isfinite(gr.float()).all() and torch.count_nonzero(gr) > 0, path_
