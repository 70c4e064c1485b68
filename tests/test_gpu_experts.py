"""GPU parity of the full-expert layer (MoE_CMix, moe.py:170-242) through
rwkvmoe_experts_forward against the oracle's dense expert loop: router
logits and indices bit-exact, dispatch bit-exact, the output within the
dtype tolerance (1e-5 fp32, 2e-2 fp16 / bf16), aux and z within 1e-5.
Shapes: small layers in each dtype (one with a carried shift state and a
residual), a single expert, a ragged top-3 layer, a skewed E = 32 top-4
layer with a logit bias, and the D = 768, E = 8 layer at 4096 tokens
(checked on sampled rows).  Also: the torch module with the reference's
parameter names runs the same computation."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import TOL, assert_close, sample_rows, to_dev, to_np
from oracle import moe_oracle as O
from rwkv_mlx_amd.workloads import zipf_bias

pytestmark = pytest.mark.gpu

# name: (dtype, B, T, C, F, E, k, x_prev, bias, residual)
CASES = {
    "exp-c128-e4-k2-f16": ("f16", 2, 24, 128, 256, 4, 2, False, False, False),
    "exp-c128-e4-k2-bf16-prev-resid": ("bf16", 2, 24, 128, 256, 4, 2, True, False, True),
    "exp-c64-e1-k1-f32": ("f32", 1, 40, 64, 128, 1, 1, False, False, False),
    "exp-ragged-e5-k3-f32": ("f32", 3, 37, 128, 256, 5, 3, True, False, False),
    "exp-skew-e32-k4-f16": ("f16", 4, 256, 256, 512, 32, 4, False, True, False),
    "exp-d768-e8-k2-f16": ("f16", 8, 512, 768, 3072, 8, 2, False, False, False),
    "exp-e64-k8-f16": ("f16", 2, 40, 192, 320, 64, 8, False, False, False),
    "exp-decode-e8-k2-f32": ("f32", 33, 1, 128, 256, 8, 2, True, False, False),
}
FULL_ORACLE_TOKENS = 1024


def _inputs(dtype, B, T, C, F, E, xp, bias, resid, seed):
    rng = np.random.default_rng(seed)
    r = lambda a: O.round_to(a, dtype)
    g = {"x": r(rng.standard_normal((B, T, C))), "x_k": r(rng.uniform(0, 1, (E, C))),
         "Wk": r(rng.standard_normal((E, F, C)) / np.sqrt(C)), "Wv": r(rng.standard_normal((E, C, F)) / np.sqrt(F)),
         "Wg": r(rng.standard_normal((E, C)) / np.sqrt(C))}
    if xp:
        g["x_prev"] = r(rng.standard_normal((B, C)))
    if bias:
        g["bias"] = zipf_bias(E, 1.2, 1.0)
    if resid:
        g["residual"] = r(rng.standard_normal((B, T, C)))
    return g


@pytest.fixture(scope="module", params=list(CASES))
def case(request, device):
    import torch
    from rwkv_mlx_amd import _lib
    name = request.param
    print(f"\n[experts case] {name}", flush=True)
    dtype, B, T, C, F, E, k, xp, bias, resid = CASES[name]
    g = _inputs(dtype, B, T, C, F, E, xp, bias, resid, seed=5000 + list(CASES).index(name))
    N = B * T
    dev = device
    up = lambda a: to_dev(a, dtype, dev)
    flags = (_lib.HAS_PREV if xp else 0) | (_lib.HAS_BIAS if bias else 0) | (_lib.ADD_RESIDUAL if resid else 0)
    desc = _lib.make_desc(B, T, C, F, E, k, 1, dtype, _lib.MODE_FUSED, flags)
    nbytes = _lib.experts_workspace_bytes(desc)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    x = up(g["x"])
    out = torch.empty_like(x)
    losses = torch.empty(2, dtype=torch.float32, device=dev)
    ex = dict(logits=torch.empty(N, E, dtype=torch.float32, device=dev),
              inds=torch.empty(N, k, dtype=torch.int32, device=dev),
              perm=torch.empty(N * k, dtype=torch.int32, device=dev),
              offsets=torch.empty(E + 1, dtype=torch.int32, device=dev))
    t = _lib.make_tensors(x=x, x_prev=up(g["x_prev"]) if xp else None, x_k=up(g["x_k"]), w_key=up(g["Wk"]),
                          w_value=up(g["Wv"]), w_gate=up(g["Wg"]),
                          logit_bias=torch.from_numpy(g["bias"]).to(dev) if bias else None,
                          residual=up(g["residual"]) if resid else None, out=out, losses=losses, **ex)
    _lib.call("rwkvmoe_experts_forward", desc, t, ws, nbytes, _lib.current_stream(dev))
    torch.cuda.synchronize()
    rt = O.router(g["x"].reshape(N, C), g["Wg"], k, dtype, g.get("bias"))
    rows = np.arange(N) if N <= FULL_ORACLE_TOKENS else sample_rows(N, T, n=128)
    ref = O.experts_rows(g["x"], g, k, dtype, rows, rt, x_prev=g.get("x_prev"))
    if resid:
        ref = O.round_to(g["residual"].reshape(N, C)[rows] + ref, dtype)
    return dict(g=g, out=to_np(out).reshape(N, C), losses=losses.cpu().numpy(), ex=ex, rt=rt, rows=rows, ref=ref,
                dtype=dtype, E=E, k=k, N=N, name=name)


def test_router_and_dispatch_bitexact(case):
    rt, ex = case["rt"], case["ex"]
    assert np.array_equal(ex["logits"].cpu().numpy().view(np.uint32), rt["logits"].astype(np.float32).view(np.uint32))
    assert np.array_equal(ex["inds"].cpu().numpy(), rt["inds"])
    p, _, o = O.dispatch(rt["inds"], case["E"])
    assert np.array_equal(ex["perm"].cpu().numpy(), p)
    assert np.array_equal(ex["offsets"].cpu().numpy(), o)
    l = case["losses"]
    assert abs(l[0] - rt["aux"]) <= 1e-5 * abs(rt["aux"]) + 1e-7
    assert abs(l[1] - rt["z"]) <= 1e-5 * abs(rt["z"]) + 1e-7


def test_output_matches_dense_expert_loop(case):
    got = case["out"]
    assert np.all(np.isfinite(got))
    assert_close(got[case["rows"]], case["ref"], case["dtype"], case["name"])


def test_small_layer_against_the_literal_dense_loop(device):
    """The oracle's literal dense loop over all experts (no row selection)."""
    c = ("f16", 1, 32, 64, 128, 3, 2)
    dtype, B, T, C, F, E, k = c
    g = _inputs(dtype, B, T, C, F, E, False, False, False, seed=77)
    import torch
    from rwkv_mlx_amd import MoE_CMix, RWKVConfig
    m = MoE_CMix(RWKVConfig(n_embd=C, dim_ffn=F), 0, E, k).to(device=device, dtype=torch.float16)
    with torch.no_grad():
        m.x_k.copy_(to_dev(g["x_k"], dtype, device).reshape(E, 1, 1, C))
        m.expert_key.copy_(to_dev(g["Wk"], dtype, device))
        m.expert_val.copy_(to_dev(g["Wv"], dtype, device))
        m.router.gate.weight.copy_(to_dev(g["Wg"], dtype, device))
    out_g, _, _ = m(to_dev(g["x"], dtype, device))  # recorded by autograd (the experts backward)
    assert out_g.requires_grad
    with torch.no_grad():
        out, aux, z = m(to_dev(g["x"], dtype, device))
    assert torch.equal(out_g.detach(), out)
    ref, raux, rz = O.experts_forward(g["x"], g, k, dtype)
    assert_close(to_np(out).reshape(-1, C), ref.reshape(-1, C), dtype, "module")
    assert abs(float(aux) - raux) <= 1e-5 * abs(raux) and abs(float(z) - rz) <= 1e-5 * abs(rz)
    assert [n for n, _ in m.named_parameters()] == ["x_k", "expert_key", "expert_val", "router.gate.weight"]
    assert float(m.orthogonal_loss()) == 0.0
