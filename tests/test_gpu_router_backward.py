"""GPU parity of the standalone Router's VJP (rwkvmoe_router_backward, the
reference's differentiable Router of rwkv_mlx/moe.py:35-86) against the
float64 oracle (oracle/moe_backward.router_backward, pinned by finite
differences in tests/test_backward_oracle.py), through the C ABI and through
torch autograd on the module.

Bars: d_x and d_w_gate within 1e-5 (fp32) / 2e-2 (fp16, bf16) relative, both
max-rel and norm-rel (helpers.TOL); two calls bit-identical; a NULL gradient
is not written.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import TOL, assert_close, to_dev, to_np
from oracle import moe_backward as MB
from oracle import moe_oracle as O
from rwkv_mlx_amd.workloads import zipf_bias

pytestmark = pytest.mark.gpu

# (name, N, C, E, k, dtype, zipf bias)
CASES = [
    ("d768-e8-k2-f16-4096", 4096, 768, 8, 2, "f16", False),
    ("d512-e4-k1-f32-512", 512, 512, 4, 1, "f32", False),
    ("d2048-e16-k2-bf16-1024", 1024, 2048, 16, 2, "bf16", False),
    ("d1024-e32-k4-f16-zipf", 1024, 1024, 32, 4, "f16", True),
    ("d192-e64-k8-f32-200", 200, 192, 64, 8, "f32", False),
]
IDS = [c[0] for c in CASES]


def _inputs(N, C, E, k, dtype, zipf, seed):
    rng = np.random.default_rng(seed)
    x = O.round_to(rng.standard_normal((N, C)), dtype)
    Wg = O.round_to(rng.standard_normal((E, C)) / np.sqrt(C), dtype)
    dg = O.round_to(rng.standard_normal((N, k)), dtype)
    bias = zipf_bias(E, 1.2) if zipf else None
    return x, Wg, dg, bias


def _run(device, x, Wg, dg, bias, k, dtype, d_losses=(0.3, 0.7), want=("d_x", "d_w_gate")):
    import torch
    from rwkv_mlx_amd import _lib
    N, C = x.shape
    E = Wg.shape[0]
    xd, wd, gd = to_dev(x, dtype, device), to_dev(Wg, dtype, device), to_dev(dg, dtype, device)
    bd = torch.from_numpy(bias).to(device) if bias is not None else None
    flags = _lib.HAS_BIAS if bias is not None else 0
    desc = _lib.make_desc(1, N, C, 64, E, k, 1, dtype, _lib.MODE_FUSED, flags)
    nb = _lib.workspace_bytes(desc)
    ws = torch.empty(nb, dtype=torch.uint8, device=device)
    logits = torch.empty(N, E, dtype=torch.float32, device=device)
    inds = torch.empty(N, k, dtype=torch.int32, device=device)
    gates = torch.empty(N, k, dtype=xd.dtype, device=device)
    losses = torch.empty(2, dtype=torch.float32, device=device)
    st = _lib.current_stream(device)
    t = _lib.make_tensors(x=xd, w_gate=wd, logit_bias=bd, logits=logits, inds=inds, gates=gates, losses=losses)
    _lib.call("rwkvmoe_router_topk", desc, t, ws, nb, st)
    out = {}
    if "d_x" in want:
        out["d_x"] = torch.full_like(xd, float("nan"))
    if "d_w_gate" in want:
        out["d_w_gate"] = torch.full_like(wd, float("nan"))
    bn = _lib.router_backward_workspace_bytes(desc)
    bws = torch.empty(bn, dtype=torch.uint8, device=device)
    dl = torch.tensor(d_losses, dtype=torch.float32, device=device)
    _lib.router_backward(desc, bws, bn, st, x=xd, w_gate=wd, logits=logits, inds=inds, d_gates=gd, d_losses=dl,
                         **out)
    torch.cuda.synchronize()
    return out, inds.cpu().numpy()


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_router_backward_matches_oracle(device, case):
    name, N, C, E, k, dtype, zipf = case
    print(f"\n[router backward] {name}", flush=True)
    x, Wg, dg, bias = _inputs(N, C, E, k, dtype, zipf, seed=1000 + IDS.index(name))
    got, inds = _run(device, x, Wg, dg, bias, k, dtype)
    ref = MB.router_backward(x, Wg, k, dtype, dg, 0.3, 0.7, bias)
    assert np.array_equal(inds, ref["inds"]), "the forward's selection differs from the oracle's"
    assert_close(to_np(got["d_x"]), ref["dx"], dtype, f"{name} d_x")
    assert_close(to_np(got["d_w_gate"]), ref["dWg"], dtype, f"{name} d_w_gate")


def test_router_backward_deterministic_and_null_outputs(device):
    x, Wg, dg, bias = _inputs(2048, 768, 8, 2, "f16", False, seed=9)
    a, _ = _run(device, x, Wg, dg, bias, 2, "f16")
    b, _ = _run(device, x, Wg, dg, bias, 2, "f16")
    for n in a:
        assert np.array_equal(to_np(a[n]).view(np.uint32), to_np(b[n]).view(np.uint32)), n
    only_w, _ = _run(device, x, Wg, dg, bias, 2, "f16", want=("d_w_gate",))
    assert np.array_equal(to_np(only_w["d_w_gate"]), to_np(a["d_w_gate"]))
    # losses only (no gate cotangent): aux and z terms alone
    got, _ = _run(device, x, Wg, np.zeros_like(dg), bias, 2, "f16")
    ref = MB.router_backward(x, Wg, 2, "f16", np.zeros_like(dg), 0.3, 0.7)
    assert_close(to_np(got["d_w_gate"]), ref["dWg"], "f16", "losses-only d_w_gate")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_router_module_autograd(device, dtype):
    """torch autograd through Router: gradients of <w, gates> + 0.3·aux +
    0.7·z reach x and gate.weight, equal to the oracle's VJP."""
    import torch
    from rwkv_mlx_amd.moe import Router
    from helpers import torch_dtype
    N, C, E, k = 600, 512, 8, 2
    x, Wg, dg, _ = _inputs(N, C, E, k, dtype, False, seed=31)
    r = Router(C, E, k).to(device=device, dtype=torch_dtype(dtype))
    with torch.no_grad():
        r.gate.weight.copy_(to_dev(Wg, dtype, device))
    xd = to_dev(x, dtype, device).reshape(2, N // 2, C).requires_grad_(True)
    inds, gates, aux, z = r(xd)
    w = to_dev(dg, dtype, device).reshape(2, N // 2, k)
    loss = (gates.float() * w.float()).sum() + 0.3 * aux + 0.7 * z
    loss.backward()
    ref = MB.router_backward(x, Wg, k, dtype, dg, 0.3, 0.7)
    assert np.array_equal(inds.reshape(N, k).cpu().numpy(), ref["inds"])
    assert_close(to_np(xd.grad).reshape(N, C), ref["dx"], dtype, "module d_x")
    assert_close(to_np(r.gate.weight.grad), ref["dWg"], dtype, "module d_w_gate")
    assert TOL[dtype] > 0
