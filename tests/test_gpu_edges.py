"""GPU parity on edge shapes and inputs, through the C ABI, against the oracle.

Shapes: a ragged token count with odd E, k, r; the smallest layer (C = F =
64, one expert, top-1, rank 1); the largest expert count, top-k and rank
(E = 64, k = 8, r = 32); top-k equal to E in fp32; a wide d_model that
shrinks the router's token tile; 1000 tokens at top-3, whose dispatch
workgroups (240 assignments each) end off a 256 boundary; adapter column
tiles (E·r > 128) with ranks 5 and 6, whose 4-column epilogue groups can
straddle two experts.  Inputs: exactly
tied router logits (duplicate gate rows: the lower expert id must win),
every token routed to one expert (a bias far above the logits), and a batch
of single-token sequences with a carried shift state.  Each case checks router logits,
indices and dispatch bit-exactly, and the forward in both modes within the
dtype's tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import Layer, assert_close, oracle_rows, to_np
from oracle import moe_oracle as O
from rwkv_mlx_amd.workloads import LayerShape, make_inputs

pytestmark = pytest.mark.gpu

CASES = {
    "ragged-e5-k3-r3-f16": LayerShape("ragged-e5-k3-r3-f16", "f16", 3, 37, 128, 256, 5, 3, 3, seed=7001),
    "min-c64-e1-k1-r1-bf16": LayerShape("min-c64-e1-k1-r1-bf16", "bf16", 1, 1, 64, 64, 1, 1, 1, seed=7002),
    "max-e64-k8-r32-f16": LayerShape("max-e64-k8-r32-f16", "f16", 2, 5, 192, 320, 64, 8, 32, seed=7003),
    "topk-eq-e-f32": LayerShape("topk-eq-e-f32", "f32", 1, 17, 64, 128, 2, 2, 16, seed=7004),
    "wide-c4096-f16": LayerShape("wide-c4096-f16", "f16", 1, 24, 4096, 256, 4, 2, 8, seed=7005),
    "decode-e16-k2-bf16": LayerShape("decode-e16-k2-bf16", "bf16", 19, 1, 256, 512, 16, 2, 16, decode=True, seed=7006),
    # the decode batch at D = 768: its key product (64 x 3200 with the adapter
    # columns) runs 64x16 tiles over the whole K, no split
    "decode-d768-e8-k2-f16": LayerShape("decode-d768-e8-k2-f16", "f16", 64, 1, 768, 3072, 8, 2, 16, decode=True,
                                        seed=7007),
    # 3000 top-3 assignments: the sparse dispatch takes the router's counts of
    # 16-token blocks (48 assignments) as histograms, 5 blocks (240) a
    # workgroup, the last one ragged
    "ragged-n1000-e6-k3-f16": LayerShape("ragged-n1000-e6-k3-f16", "f16", 1, 1000, 128, 256, 6, 3, 8, seed=7009),
    # 16384 tokens at top-4 over a 64-wide FFN: the SPARSE forward's dispatch
    # job has 256 blocks of 256 assignments and the key GEMM's launch 128
    # workgroups (128x64 tiles), so workgroups take several blocks by ticket
    "many-blocks-f64-e4-k4-f16": LayerShape("many-blocks-f64-e4-k4-f16", "f16", 8, 2048, 128, 64, 4, 4, 8, seed=7010),
    # E·r > 128 with a rank that is not a multiple of 4: the adapter column
    # tiles' epilogue meets 4-column groups that straddle two experts (2048
    # tokens on 128-row tiles, and 9 tokens whose key product splits K)
    "adtiles-e30-k2-r5-f16": LayerShape("adtiles-e30-k2-r5-f16", "f16", 2, 1024, 256, 512, 30, 2, 5, seed=7011),
    "adtiles-e24-k2-r6-bf16": LayerShape("adtiles-e24-k2-r6-bf16", "bf16", 1, 9, 512, 256, 24, 2, 6, seed=7012),
}


def _ties(g):
    """Gate rows 1 and 2 identical, and row 4 = row 0: tied logits."""
    g = dict(g)
    wg = g["Wg"].copy()
    wg[2] = wg[1]
    wg[4] = wg[0]
    g["Wg"] = wg
    return g


def _collapse(g):
    """A bias far above every logit on expert 3: all tokens pick it first
    (small enough that exp of the logits stays finite)."""
    g = dict(g)
    E = g["Wg"].shape[0]
    b = np.zeros(E, np.float32)
    b[3] = 30.0
    g["bias"] = b
    return g


INPUT_CASES = {
    "ties-e6-k2-f16": (LayerShape("ties-e6-k2-f16", "f16", 2, 48, 128, 256, 6, 2, 8, seed=7007), _ties),
    "collapse-e8-k2-f16": (LayerShape("collapse-e8-k2-f16", "f16", 2, 40, 128, 256, 8, 2, 16, seed=7008), _collapse),
}


def _layer(shape, device, transform=None):
    g = make_inputs(shape)
    if transform is not None:
        g = transform(g)
    L = Layer(shape, device, inputs=g)
    if "bias" in g and L.bias is None:  # a transform added a bias
        import torch
        from rwkv_mlx_amd import _lib
        L.bias = torch.from_numpy(g["bias"]).to(device)
        L.flags |= _lib.HAS_BIAS
        L.desc = L.make_desc()
    L.router_ref = O.router(g["x"].reshape(L.N, -1), g["Wg"], shape.top_k, shape.dtype, g.get("bias"))
    L.rows = np.arange(L.N)
    L.ref = oracle_rows(g, shape, L.rows, L.router_ref)
    return L


@pytest.fixture(scope="module", params=list(CASES) + list(INPUT_CASES))
def layer(request, device):
    print(f"\n[edge case] {request.param}", flush=True)
    if request.param in CASES:
        return _layer(CASES[request.param], device)
    shape, tf = INPUT_CASES[request.param]
    return _layer(shape, device, tf)


def _router(L):
    import torch
    w = L.w
    logits = torch.empty(L.N, w.n_experts, dtype=torch.float32, device=L.dev)
    inds = torch.empty(L.N, w.top_k, dtype=torch.int32, device=L.dev)
    gates = torch.empty(L.N, w.top_k, dtype=L.dt, device=L.dev)
    losses = torch.empty(2, dtype=torch.float32, device=L.dev)
    L.call("rwkvmoe_router_topk", x=L.x, w_gate=L.Wg, logit_bias=L.bias, logits=logits, inds=inds, gates=gates,
           losses=losses)
    torch.cuda.synchronize()
    return to_np(logits), inds.cpu().numpy(), losses.cpu().numpy()


def test_router_and_dispatch_bitexact(layer):
    L = layer
    ref = L.router_ref
    logits, inds, losses = _router(L)
    assert np.array_equal(logits.view(np.uint32), ref["logits"].astype(np.float32).view(np.uint32))
    assert np.array_equal(inds, ref["inds"])
    assert np.array_equal(inds, O.topk_canonical(logits, L.w.top_k))
    assert abs(losses[0] - ref["aux"]) <= 1e-5 * abs(ref["aux"]) + 1e-7
    assert abs(losses[1] - ref["z"]) <= 1e-5 * abs(ref["z"]) + 1e-7


@pytest.mark.parametrize("mode", ["fused", "sparse"])
def test_forward(layer, mode):
    L = layer
    out, losses, ex = L.forward(mode=mode, extras=True)
    base_ref, delta_ref, out_ref, r = L.ref
    assert_close(to_np(out).reshape(L.N, -1), out_ref, L.w.dtype, f"{L.w.name}/{mode}")
    assert np.array_equal(ex["inds"].cpu().numpy(), r["inds"])
    p, i, o = O.dispatch(r["inds"], L.w.n_experts)
    assert np.array_equal(ex["perm"].cpu().numpy(), p)
    assert np.array_equal(ex["inv_perm"].cpu().numpy(), i)
    assert np.array_equal(ex["offsets"].cpu().numpy(), o)
    l = losses.cpu().numpy()
    assert abs(l[0] - r["aux"]) <= 1e-5 * abs(r["aux"]) + 1e-7
    assert abs(l[1] - r["z"]) <= 1e-5 * abs(r["z"]) + 1e-7


def test_run_twice_bit_identical(layer):
    for mode in ("fused", "sparse"):
        a, la, _ = layer.forward(mode=mode)
        b, lb, _ = layer.forward(mode=mode)
        assert np.array_equal(to_np(a), to_np(b)), mode
        assert np.array_equal(la.cpu().numpy(), lb.cpu().numpy()), mode


def test_ties_pick_lower_id(device):
    shape, tf = INPUT_CASES["ties-e6-k2-f16"]
    L = _layer(shape, device, tf)
    logits, inds, _ = _router(L)
    assert np.array_equal(logits[:, 1].view(np.uint32), logits[:, 2].view(np.uint32))
    # wherever expert 2 is chosen its tied twin 1 is chosen too, in an earlier slot
    for t in range(L.N):
        row = list(inds[t])
        if 2 in row:
            assert 1 in row and row.index(1) < row.index(2)


def test_collapse_routes_everything_to_one_expert(device):
    shape, tf = INPUT_CASES["collapse-e8-k2-f16"]
    L = _layer(shape, device, tf)
    _, inds, _ = _router(L)
    assert np.all(inds[:, 0] == 3)
    _, _, ex = L.forward(mode="sparse", extras=True)
    offs = ex["offsets"].cpu().numpy()
    assert offs[4] - offs[3] == L.N  # expert 3 holds one assignment per token
