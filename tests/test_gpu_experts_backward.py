"""GPU parity of the full-expert backward (rwkvmoe_experts_backward, through
the C ABI) against the float64 oracle (oracle/moe_backward.py
``experts_backward``, itself pinned by finite differences and torch float64
autograd), and of the torch autograd path of MoE_CMix.

Each case runs rwkvmoe_experts_forward (for the logits and selection it
saves; the selection is checked bit-exact against the oracle's router), then
the backward with a seeded d_out and non-zero aux / z cotangents, and checks
d_x, d_x_prev (with a carried state), d_x_k, d_w_key, d_w_value and
d_w_gate.  Tolerance (max|got-ref| / max|ref| and the 2-norm ratio): 1e-5
for fp32 layers, 2e-2 for fp16 / bf16 (the intermediate products are
rounded to the layer dtype, as MLX's fp16 / bf16 VJPs round them).  Also:
two runs are bit-identical; outputs left NULL change nothing else; with
expert_val = 0, x_k and expert_key get exactly zero gradient.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import to_dev, to_np, torch_dtype
from oracle import moe_backward as MB
from oracle import moe_oracle as O
from rwkv_mlx_amd.workloads import zipf_bias

pytestmark = pytest.mark.gpu

BWD_TOL = {"f32": 1e-5, "f16": 2e-2, "bf16": 2e-2}
D_LOSSES = (0.3, -0.7)
GRADS = ("d_x", "d_x_prev", "d_x_k", "d_w_key", "d_w_value", "d_w_gate")
ORACLE_NAME = {"d_x": "dx", "d_x_prev": "dx_prev", "d_x_k": "dx_k", "d_w_key": "dWk", "d_w_value": "dWv",
               "d_w_gate": "dWg"}

# name: (dtype, B, T, C, F, E, k, x_prev, bias)
CASES = {
    "xbwd-c128-e4-k2-f32-prev-bias": ("f32", 2, 24, 128, 256, 4, 2, True, True),
    "xbwd-c128-e4-k2-f16-prev": ("f16", 2, 24, 128, 256, 4, 2, True, False),
    "xbwd-c128-e4-k2-bf16": ("bf16", 2, 24, 128, 256, 4, 2, False, False),
    "xbwd-ragged-e5-k3-f32-prev": ("f32", 3, 37, 128, 256, 5, 3, True, False),
    "xbwd-e1-k1-bf16": ("bf16", 1, 40, 64, 128, 1, 1, False, False),
    "xbwd-d768-e8-k2-f16": ("f16", 1, 256, 768, 3072, 8, 2, False, False),
    "xbwd-e64-k8-f16": ("f16", 2, 40, 192, 320, 64, 8, False, False),
    "xbwd-skew-e32-k4-f32-bias": ("f32", 1, 96, 256, 512, 32, 4, False, True),
    "xbwd-decode-e8-k2-bf16-prev": ("bf16", 64, 1, 256, 512, 8, 2, True, False),
}


def _errs(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    mx = max(float(np.max(np.abs(ref))), 1e-30)
    nrm = max(float(np.linalg.norm(ref)), 1e-30)
    return float(np.max(np.abs(got - ref))) / mx, float(np.linalg.norm(got - ref)) / nrm


def _bits(t):
    import torch
    return t.detach().contiguous().view(-1).view(torch.uint8).cpu().numpy()


class ExpertsLayer:
    """One full-expert layer's inputs on the device, forward and backward
    through the C ABI."""

    def __init__(self, name, device, zero_values=False):
        import torch
        from rwkv_mlx_amd import _lib
        dtype, B, T, C, F, E, k, xp, bias = CASES[name]
        self.name, self.dtype, self.dev = name, dtype, device
        self.B, self.T, self.C, self.F, self.E, self.k, self.N = B, T, C, F, E, k, B * T
        rng = np.random.default_rng(9100 + list(CASES).index(name))
        r = lambda a: O.round_to(a, dtype)
        g = {"x": r(rng.standard_normal((B, T, C))), "x_k": r(rng.uniform(0, 1, (E, C))),
             "Wk": r(rng.standard_normal((E, F, C)) / np.sqrt(C)),
             "Wv": r(rng.standard_normal((E, C, F)) / np.sqrt(F)),
             "Wg": r(rng.standard_normal((E, C)) / np.sqrt(C))}
        if zero_values:
            g["Wv"][:] = 0
        g["x_prev"] = r(rng.standard_normal((B, C))) if xp else None
        g["bias"] = zipf_bias(E, 1.2, 1.0) if bias else None
        g["dO"] = r(rng.standard_normal((B, T, C)))
        self.g = g
        self.dt = torch_dtype(dtype)
        up = lambda a: None if a is None else to_dev(a, dtype, device)
        self.x, self.xp, self.xk = up(g["x"]), up(g["x_prev"]), up(g["x_k"])
        self.Wk, self.Wv, self.Wg, self.dO = up(g["Wk"]), up(g["Wv"]), up(g["Wg"]), up(g["dO"])
        self.bias = torch.from_numpy(g["bias"]).to(device) if bias else None
        self.flags = (_lib.HAS_PREV if xp else 0) | (_lib.HAS_BIAS if bias else 0)
        self.desc = _lib.make_desc(B, T, C, F, E, k, 1, dtype, _lib.MODE_FUSED, self.flags)
        self.d_losses = torch.tensor(D_LOSSES, dtype=torch.float32, device=device)
        self.shapes = {"d_x": (B, T, C), "d_x_prev": (B, C), "d_x_k": (E, C), "d_w_key": (E, F, C),
                       "d_w_value": (E, C, F), "d_w_gate": (E, C)}

    def forward(self):
        import torch
        from rwkv_mlx_amd import _lib
        nbytes = _lib.experts_workspace_bytes(self.desc)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=self.dev)
        out = torch.empty_like(self.x)
        losses = torch.empty(2, dtype=torch.float32, device=self.dev)
        self.logits = torch.empty(self.N, self.E, dtype=torch.float32, device=self.dev)
        self.inds = torch.empty(self.N, self.k, dtype=torch.int32, device=self.dev)
        t = _lib.make_tensors(x=self.x, x_prev=self.xp, x_k=self.xk, w_key=self.Wk, w_value=self.Wv, w_gate=self.Wg,
                              logit_bias=self.bias, out=out, losses=losses, logits=self.logits, inds=self.inds)
        _lib.call("rwkvmoe_experts_forward", self.desc, t, ws, nbytes, _lib.current_stream(self.dev))
        torch.cuda.synchronize()
        return out, losses

    def backward(self, outputs=GRADS):
        import torch
        from rwkv_mlx_amd import _lib
        outs = {n: torch.full(self.shapes[n], float("nan"), dtype=self.dt, device=self.dev) for n in outputs
                if n != "d_x_prev" or self.xp is not None}
        nbytes = _lib.experts_backward_workspace_bytes(self.desc)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=self.dev)
        _lib.experts_backward(self.desc, ws, nbytes, _lib.current_stream(self.dev), x=self.x, x_prev=self.xp,
                              x_k=self.xk, w_key=self.Wk, w_value=self.Wv, w_gate=self.Wg, logits=self.logits,
                              inds=self.inds, d_out=self.dO, d_losses=self.d_losses, **outs)
        torch.cuda.synchronize()
        return outs

    def oracle(self):
        g = self.g
        p = {"x_k": g["x_k"], "Wk": g["Wk"], "Wv": g["Wv"], "Wg": g["Wg"]}
        return MB.experts_backward(g["x"], p, self.k, self.dtype, g["dO"], D_LOSSES[0], D_LOSSES[1],
                                   x_prev=g["x_prev"], bias=g["bias"])


@pytest.fixture(scope="module", params=list(CASES))
def case(request, device):
    name = request.param
    print(f"\n[experts backward case] {name}", flush=True)
    L = ExpertsLayer(name, device)
    L.forward()
    ref = L.oracle()
    return L, ref


def test_selection_matches_oracle(case):
    L, ref = case
    assert np.array_equal(L.inds.cpu().numpy(), ref["inds"])


def test_gradients_match_oracle(case):
    L, ref = case
    outs = L.backward()
    tol = BWD_TOL[L.dtype]
    for name, got in outs.items():
        g = to_np(got)
        want = np.asarray(ref[ORACLE_NAME[name]]).reshape(g.shape)
        assert np.all(np.isfinite(g)), f"{L.name} {name}: non-finite"
        emax, enorm = _errs(g, want)
        assert emax <= tol and enorm <= tol, f"{L.name} {name}: max-rel {emax:.3e} norm-rel {enorm:.3e} > {tol}"


def test_backward_is_deterministic_and_null_outputs_skip(case):
    L, _ = case
    a = L.backward()
    b = L.backward()
    for n in a:
        assert np.array_equal(_bits(a[n]), _bits(b[n])), n
    only = L.backward(outputs=("d_w_value",))
    assert np.array_equal(_bits(only["d_w_value"]), _bits(a["d_w_value"]))
    some = L.backward(outputs=("d_x", "d_w_gate"))
    for n in some:
        assert np.array_equal(_bits(some[n]), _bits(a[n])), n


def test_zero_values_give_zero_key_gradients(device):
    L = ExpertsLayer("xbwd-c128-e4-k2-f16-prev", device, zero_values=True)
    L.forward()
    outs = L.backward()
    assert np.all(to_np(outs["d_x_k"]) == 0) and np.all(to_np(outs["d_w_key"]) == 0)
    assert np.all(to_np(outs["d_x_prev"]) == 0)
    ref = L.oracle()
    for n in ("d_x", "d_w_value", "d_w_gate"):
        emax, enorm = _errs(to_np(outs[n]), np.asarray(ref[ORACLE_NAME[n]]).reshape(outs[n].shape))
        assert emax <= BWD_TOL["f16"] and enorm <= BWD_TOL["f16"], n


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_module_autograd_matches_oracle(device, dtype):
    """MoE_CMix under autograd: out·dO + d_aux·aux + d_z·z backpropagated
    through the module reaches every parameter, x and x_prev."""
    import torch
    from rwkv_mlx_amd import MoE_CMix, RWKVConfig
    B, T, C, F, E, k = 2, 20, 128, 256, 4, 2
    rng = np.random.default_rng(77 if dtype == "f32" else 78)
    r = lambda a: O.round_to(a, dtype)
    g = {"x": r(rng.standard_normal((B, T, C))), "x_k": r(rng.uniform(0, 1, (E, C))),
         "Wk": r(rng.standard_normal((E, F, C)) / np.sqrt(C)), "Wv": r(rng.standard_normal((E, C, F)) / np.sqrt(F)),
         "Wg": r(rng.standard_normal((E, C)) / np.sqrt(C)), "x_prev": r(rng.standard_normal((B, C))),
         "dO": r(rng.standard_normal((B, T, C)))}
    dt = torch_dtype(dtype)
    m = MoE_CMix(RWKVConfig(n_embd=C, dim_ffn=F), 0, E, k).to(device=device, dtype=dt)
    with torch.no_grad():
        m.x_k.copy_(to_dev(g["x_k"], dtype, device).reshape(E, 1, 1, C))
        m.expert_key.copy_(to_dev(g["Wk"], dtype, device))
        m.expert_val.copy_(to_dev(g["Wv"], dtype, device))
        m.router.gate.weight.copy_(to_dev(g["Wg"], dtype, device))
    x = to_dev(g["x"], dtype, device).requires_grad_(True)
    xp = to_dev(g["x_prev"], dtype, device).requires_grad_(True)
    out, aux, z = m(x, x_prev=xp)
    with torch.no_grad():
        out0, aux0, z0 = m(x, x_prev=xp)
    assert np.array_equal(_bits(out), _bits(out0)) and float(aux.detach()) == float(aux0) and float(z.detach()) == float(z0)
    loss = (out.float() * to_dev(g["dO"], dtype, device).float()).sum() + D_LOSSES[0] * aux + D_LOSSES[1] * z
    loss.backward()
    p = {"x_k": g["x_k"], "Wk": g["Wk"], "Wv": g["Wv"], "Wg": g["Wg"]}
    ref = MB.experts_backward(g["x"], p, k, dtype, g["dO"], D_LOSSES[0], D_LOSSES[1], x_prev=g["x_prev"])
    pairs = [(x.grad, ref["dx"]), (xp.grad, ref["dx_prev"]), (m.x_k.grad.reshape(E, C), ref["dx_k"]),
             (m.expert_key.grad, ref["dWk"]), (m.expert_val.grad, ref["dWv"]),
             (m.router.gate.weight.grad, ref["dWg"])]
    tol = BWD_TOL[dtype]
    for i, (got, want) in enumerate(pairs):
        assert got is not None, i
        emax, enorm = _errs(to_np(got), np.asarray(want).reshape(got.shape))
        assert emax <= tol and enorm <= tol, f"grad {i}: max-rel {emax:.3e} norm-rel {enorm:.3e}"
