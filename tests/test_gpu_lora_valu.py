"""GPU parity of the grouped LoRA products on the vector ALUs
(RWKVMOE_LORA_VALU, lora_grouped_valu_kernel: v_dot2 into fp32 instead of
MFMA blocks), the alternative the SPARSE mode's kernel choice is measured
against.  The SPARSE forward with the flag matches the oracle at the dtype
tolerance (1e-5 fp32, 2e-2 fp16 / bf16) on sampled rows, and the adapter
rows of the stage entry point (rwkvmoe_lora_grouped) match the oracle's
(x·A_e)·B_e rows; routing is unaffected (bit-exact indices).
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import Layer, assert_close, oracle_rows, sample_rows, to_np
from oracle import moe_oracle as O
from rwkv_mlx_amd.workloads import BY_NAME, LayerShape

pytestmark = pytest.mark.gpu

CASES = [
    LayerShape("valu-c128-e4-k2-r8-f32", "f32", 2, 24, 128, 256, 4, 2, 8, seed=9301),
    LayerShape("valu-c128-e4-k2-r8-f16", "f16", 2, 24, 128, 256, 4, 2, 8, seed=9302),
    LayerShape("valu-ragged-e5-k3-r3-bf16", "bf16", 3, 37, 128, 256, 5, 3, 3, seed=9303),
    LayerShape("valu-e64-k8-r32-f16", "f16", 2, 40, 192, 320, 64, 8, 32, seed=9304),
    LayerShape("valu-c1536-e8-k2-r16-bf16", "bf16", 1, 96, 1536, 512, 8, 2, 16, seed=9305),
    BY_NAME["cmix-d768-e8-top2-r16-fp16"],
]


@pytest.mark.parametrize("shape", CASES, ids=lambda s: s.name)
def test_sparse_forward_with_valu_lora(device, shape):
    import torch
    from rwkv_mlx_amd import _lib
    print(f"\n[valu case] {shape.name}", flush=True)
    L = Layer(shape, device, mode="sparse")
    L.flags |= _lib.LORA_VALU
    out, losses, ex = L.forward(mode="sparse", extras=True)
    N, C = L.N, shape.d_model
    rows = np.arange(N) if N <= 1024 else sample_rows(N, shape.seq_len, n=192)
    _, _, ref, rt = oracle_rows(L.np, shape, rows)
    assert np.array_equal(ex["inds"].cpu().numpy(), rt["inds"])
    assert_close(to_np(out).reshape(N, C)[rows], ref, shape.dtype, shape.name)
    # the adapter rows of the stage entry point against (x·A_e)·B_e per routed row
    perm, offsets = ex["perm"], ex["offsets"]
    ag = torch.empty(N * shape.top_k, C, dtype=L.dt, device=device)
    L.call("rwkvmoe_lora_grouped", L.make_desc(mode="sparse", flags=L.flags), x=L.x, lora_A=L.A, lora_B=L.B,
           perm=perm, offsets=offsets, adapter_rows=ag)
    torch.cuda.synchronize()
    pm = perm.cpu().numpy()
    inds = ex["inds"].cpu().numpy().reshape(-1)
    pick = np.arange(pm.size) if pm.size <= 2048 else np.random.default_rng(1).choice(pm.size, 512, replace=False)
    x = L.np["x"].reshape(-1, C)
    a, e = pm[pick], inds[pm[pick]]
    got = to_np(ag)[a]  # (rows in assignment order)
    s_e = O.round_to(np.einsum("nc,ncr->nr", x[a // shape.top_k].astype(np.float64),
                               L.np["A"][e].astype(np.float64)), shape.dtype)
    want = O.round_to(np.einsum("nr,nrc->nc", s_e.astype(np.float64), L.np["B"][e].astype(np.float64)), shape.dtype)
    assert_close(got, want, shape.dtype, shape.name + " adapter rows")


def test_valu_flag_rejected_with_fp32_adapters(device):
    from rwkv_mlx_amd import _lib
    d = _lib.make_desc(1, 64, 128, 256, 4, 2, 8, "f16", "sparse", _lib.LORA_VALU | _lib.ADAPTERS_F32)
    with pytest.raises(_lib.RwkvMoeError):
        _lib.workspace_bytes(d)
