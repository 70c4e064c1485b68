"""The SPARSE forward with the adapters on chip, where the D=768 fixtures do
not reach (moe.py:138-147).

The forward takes that form for 16-bit layers whose E·r fits one
128-column slice (r a multiple of 8), top-k <= 4 and a value product on the
128x96 tile (about 3.7K tokens and up): the router writes u = round(x·A_e)
for every expert, and the value product adds one K slice per routing rank
and combines in its epilogue.  Cases: top-1 with E·r = 64 (half the slice is
padding), 16 experts at top-4 (four rank slices), top-3 in bf16 over 4000
tokens (a ragged last row tile).  Each case checks

* which form ran: the forward's launches (rwkvmoe_forward_timed) include
  cmix_value_sparse and no grouped LoRA, and with adapter rows asked for it
  is the grouped form instead;
* routing equal to the oracle's, and out against the oracle's dense expert
  loop on sampled rows at the dtype tolerance (2e-2);
* the two forms against each other at the same tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import Layer, assert_close, oracle_rows, sample_rows, to_np
from rwkv_mlx_amd.workloads import LayerShape

pytestmark = pytest.mark.gpu

CASES = [
    LayerShape("onchip-e4-k1-r16-f16", "f16", 4, 1024, 768, 3072, 4, 1, 16, seed=9401),
    LayerShape("onchip-e16-k4-r8-f16", "f16", 4, 1024, 768, 3072, 16, 4, 8, seed=9402),
    LayerShape("onchip-e8-k3-r16-bf16", "bf16", 5, 800, 768, 3072, 8, 3, 16, seed=9403),
]


def _kernels(L, desc, tensors):
    """Names of the kernels one forward launches."""
    import torch
    from rwkv_mlx_amd import _lib
    timer = _lib.KernelTimer(torch.cuda.current_stream(L.dev), 1)
    timer.forward(desc, tensors, L.ws, L.ws_bytes)
    torch.cuda.synchronize()
    return {name for name, _ in timer.summary()}


@pytest.mark.parametrize("shape", CASES, ids=lambda s: s.name)
def test_sparse_on_chip(device, shape):
    import torch
    from rwkv_mlx_amd import _lib
    print(f"\n[sparse on chip] {shape.name}", flush=True)
    L = Layer(shape, device, mode="sparse")
    N, C, k = L.N, shape.d_model, shape.top_k
    desc = L.make_desc(mode="sparse")
    outs, names = [], []
    for rows in (False, True):
        out = torch.empty_like(L.x)
        losses = torch.empty(2, dtype=torch.float32, device=device)
        inds = torch.empty(N, k, dtype=torch.int32, device=device)
        extra = {"adapter_rows": torch.empty(N * k, C, dtype=L.dt, device=device)} if rows else {}
        t = _lib.make_tensors(out=out, losses=losses, inds=inds, **L.inputs(), **extra)
        names.append(_kernels(L, desc, t))
        outs.append((to_np(out).reshape(N, C), inds.cpu().numpy()))
    print(f"  on chip: {sorted(names[0])}\n  grouped: {sorted(names[1])}", flush=True)
    assert "cmix_value_sparse" in names[0] and "lora_grouped" not in names[0], names[0]
    assert "lora_grouped" in names[1] and "cmix_value_sparse" not in names[1], names[1]
    rows = sample_rows(N, shape.seq_len, n=192)
    rows = np.unique(np.concatenate([rows, np.arange(N - 40, N)]))  # the ragged last tile's rows
    _, _, ref, rt = oracle_rows(L.np, shape, rows)
    for (o, ind), form in zip(outs, ("on chip", "grouped")):
        assert np.array_equal(ind, rt["inds"]), f"{form}: routing differs"
        assert_close(o[rows], ref, shape.dtype, f"{shape.name} {form}")
    assert_close(outs[0][0], outs[1][0], shape.dtype, f"{shape.name} forms")
