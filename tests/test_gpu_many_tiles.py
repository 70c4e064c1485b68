"""Regression: layers whose GEMMs have more tiles than the GPU has CUs under
the 128x128 tile (the automatic choice for fp32 layers and for 16-bit
layers with d_model = 128).  That tile stages its output in the operand
ring, so each workgroup may take only one tile; the launcher now guarantees
it.  Forward parity in both modes against the oracle on sampled rows, the
router bit-exact on every row, and the backward's d_x against the backward
oracle on a token subset of the same layer shape.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import Layer, assert_close, oracle_rows, sample_rows, to_np
from oracle import moe_oracle as O
from rwkv_mlx_amd.workloads import LayerShape

pytestmark = pytest.mark.gpu

CASES = {
    # value GEMM n = C = 512 (fp32: 128x128 tiles): 16384 / 128 * 4 = 512 tiles > 256 CUs
    "tiles-c512-n16384-f32": LayerShape("tiles-c512-n16384-f32", "f32", 32, 512, 512, 2048, 4, 1, 8, seed=9001),
    # value GEMM n = C = 128 (16-bit: 128x128 tiles): 40960 / 128 = 320 tiles > 256 CUs
    "tiles-c128-n40960-f16": LayerShape("tiles-c128-n40960-f16", "f16", 40, 1024, 128, 256, 4, 2, 8, seed=9002),
}


@pytest.fixture(scope="module", params=list(CASES))
def layer(request, device):
    print(f"\n[many-tiles case] {request.param}", flush=True)
    L = Layer(CASES[request.param], device)
    g = L.np
    L.router_ref = O.router(g["x"].reshape(L.N, -1), g["Wg"], L.w.top_k, L.w.dtype, g.get("bias"))
    L.rows = sample_rows(L.N, L.w.seq_len, n=192)
    L.ref = oracle_rows(g, L.w, L.rows, L.router_ref)
    return L


@pytest.mark.parametrize("mode", ["fused", "sparse"])
def test_forward_parity_many_tiles(layer, mode):
    L = layer
    out, losses, ex = L.forward(mode=mode, extras=True)
    _, _, out_ref, r = L.ref
    full = to_np(out).reshape(L.N, -1)
    assert np.all(np.isfinite(full))
    assert_close(full[L.rows], out_ref, L.w.dtype, f"{L.w.name}/{mode}")
    assert np.array_equal(ex["logits"].cpu().numpy().view(np.uint32), r["logits"].astype(np.float32).view(np.uint32))
    assert np.array_equal(ex["inds"].cpu().numpy(), r["inds"])
