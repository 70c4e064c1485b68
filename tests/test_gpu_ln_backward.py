"""GPU parity of ln2's VJP (rwkvmoe_layer_norm_backward; the Block's
x + ffn(ln2(x)), rwkv_mlx/model.py:321, differentiated by MLX autodiff)
against the float64 oracle (oracle/moe_backward.layer_norm_backward, pinned
by torch autograd, central differences and invariants in
tests/test_layer_norm_oracle.py), through the C ABI and through torch
autograd on both modules in the Block form.

Bars: d_x, d_ln_weight and d_ln_bias within 1e-5 (fp32) / 2e-2 (fp16,
bf16) relative to the oracle, both max-rel and norm-rel (helpers.TOL).  The
column sums run in a fixed order: two calls are bit-identical, and a call
that asks for fewer outputs writes the same bits into the ones it asks for.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import TOL, assert_close, to_dev, to_np, torch_dtype
from oracle import moe_backward as MB
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

# (name, N, C, dtype, with d_res): rows held in registers (C <= 1024 for
# 16-bit, <= 512 for fp32), wide rows re-read per pass, ragged N (dead rows
# in the last workgroup), and more rows than 1024 workgroups take in one pass
CASES = [
    ("f16-4096x768-res", 4096, 768, "f16", True),
    ("bf16-1024x2048", 1024, 2048, "bf16", False),
    ("f32-512x512-res", 512, 512, "f32", True),
    ("f32-300x8192", 300, 8192, "f32", False),
    ("f16-32805x256-passes-res", 16 * 1024 * 2 + 37, 256, "f16", True),
    ("bf16-7x64", 7, 64, "bf16", False),
]
IDS = [c[0] for c in CASES]


def _inputs(N, C, dtype, seed):
    rng = np.random.default_rng(seed)
    x = O.round_to(rng.standard_normal((N, C)) * 2.0 + 0.5, dtype)
    w = O.round_to(1.0 + 0.2 * rng.standard_normal(C), dtype)
    dy = O.round_to(rng.standard_normal((N, C)), dtype)
    dr = O.round_to(rng.standard_normal((N, C)), dtype)
    return x, w, dy, dr


def _run(device, x, w, dy, dr, dtype, want=("d_x", "d_ln_weight", "d_ln_bias"), alias=False):
    import torch
    from rwkv_mlx_amd import _lib
    N, C = x.shape
    desc = _lib.make_desc(1, N, C, 64, 4, 2, 8, dtype)
    nb = _lib.layer_norm_backward_workspace_bytes(desc)
    ws = torch.empty(max(nb, 256), dtype=torch.uint8, device=device)
    xd, wd, dyd = to_dev(x, dtype, device), to_dev(w, dtype, device), to_dev(dy, dtype, device)
    drd = to_dev(dr, dtype, device) if dr is not None else None
    out = {}
    if "d_x" in want:
        out["d_x"] = dyd if alias else torch.full_like(xd, float("nan"))
    for n in ("d_ln_weight", "d_ln_bias"):
        if n in want:
            out[n] = torch.full_like(wd, float("nan"))
    _lib.layer_norm_backward(desc, ws, nb, _lib.current_stream(device), x=xd, ln_weight=wd, d_y=dyd, d_res=drd,
                             **out)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_layer_norm_backward_matches_oracle(device, case):
    name, N, C, dtype, res = case
    print(f"\n[ln backward] {name}", flush=True)
    x, w, dy, dr = _inputs(N, C, dtype, seed=2000 + IDS.index(name))
    dr = dr if res else None
    got = _run(device, x, w, dy, dr, dtype)
    ref = MB.layer_norm_backward(x, w, dy, d_res=dr)
    assert_close(to_np(got["d_x"]), ref["dx"], dtype, f"{name} d_x")
    assert_close(to_np(got["d_ln_weight"]), ref["dw"], dtype, f"{name} d_ln_weight")
    assert_close(to_np(got["d_ln_bias"]), ref["db"], dtype, f"{name} d_ln_bias")


def test_layer_norm_backward_deterministic_alias_and_subsets(device):
    x, w, dy, dr = _inputs(3000, 768, "f16", seed=11)
    a = _run(device, x, w, dy, dr, "f16")
    b = _run(device, x, w, dy, dr, "f16")
    bits = lambda t: to_np(t).view(np.uint32)
    for n in a:
        assert np.array_equal(bits(a[n]), bits(b[n])), n
    al = _run(device, x, w, dy, dr, "f16", alias=True)  # d_x written over d_y
    assert np.array_equal(bits(al["d_x"]), bits(a["d_x"]))
    only_b = _run(device, x, w, dy, dr, "f16", want=("d_ln_bias",))
    assert np.array_equal(bits(only_b["d_ln_bias"]), bits(a["d_ln_bias"]))
    only_x = _run(device, x, w, dy, dr, "f16", want=("d_x",))
    assert np.array_equal(bits(only_x["d_x"]), bits(a["d_x"]))
    assert _run(device, x, w, dy, dr, "f16", want=()) == {}


def _ln_module(C, dtype, device, seed):
    import torch
    ln = torch.nn.LayerNorm(C)
    rng = np.random.default_rng(seed)
    with torch.no_grad():
        ln.weight.copy_(torch.from_numpy(O.round_to(1.0 + 0.2 * rng.standard_normal(C), dtype)))
        ln.bias.copy_(torch.from_numpy(O.round_to(0.1 * rng.standard_normal(C), dtype)))
    return ln.to(device=device, dtype=torch_dtype(dtype))


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_lora_module_block_form_autograd(device, dtype):
    """LoRAMoE_CMix(x, residual=x, ln=ln2) under autograd — ln2 in the
    layer's launches, its VJP in rwkvmoe_layer_norm_backward with the
    residual's cotangent added there — against the oracle: the layer's VJP
    at x_ln = LN(x), its d_x rounded to the dtype (the cotangent of the
    layer input), then ln2's VJP plus dO.  Also against torch's own ln2 in
    front of the same layer (the unfused form)."""
    import torch
    from rwkv_mlx_amd.moe import build_layer
    C, F, E, k, r, B, T = 256, 512, 4, 2, 8, 2, 40
    torch.manual_seed(5)
    dt = torch_dtype(dtype)
    m = build_layer(C, F, E, k, r)
    with torch.no_grad():
        m.base.x_k.uniform_(0, 1)
        m.lora_B.normal_(0, 0.05)
    m = m.to(device=device, dtype=dt)
    ln = _ln_module(C, dtype, device, seed=6)
    rng = np.random.default_rng(7)
    x_np = O.round_to(rng.standard_normal((B, T, C)) * 1.5 + 0.3, dtype)
    dO_np = O.round_to(rng.standard_normal((B, T, C)), dtype)
    x = to_dev(x_np, dtype, device).requires_grad_(True)
    dO = to_dev(dO_np, dtype, device)
    out, aux, z = m(x, residual=x, ln=ln)
    with torch.no_grad():
        out0, _, _ = m(x, residual=x, ln=ln)
    assert torch.equal(out.detach(), out0), "the autograd forward and the inference forward differ"
    ((out.float() * dO.float()).sum() + 0.3 * aux - 0.7 * z).backward()
    f = lambda t: t.detach().float().cpu().numpy()
    N = B * T
    w, b = f(ln.weight), f(ln.bias)
    xn = O.layer_norm(x_np.reshape(N, C), w, b, dtype)
    ref = MB.moe_backward(xn, f(m.router.gate.weight), f(m.lora_A), f(m.lora_B), k, dtype, dO_np.reshape(N, C),
                          0.3, -0.7)
    lref = MB.layer_norm_backward(x_np.reshape(N, C), w, O.round_to(ref["dx"], dtype), d_res=dO_np.reshape(N, C))
    tol = TOL[dtype] if dtype != "f32" else 1e-4  # (fp32: the layer's d_x is itself within 1e-5, then ln2's VJP)
    for got, want, n in ((x.grad, lref["dx"], "dx"), (ln.weight.grad, lref["dw"], "d_ln_weight"),
                         (ln.bias.grad, lref["db"], "d_ln_bias"), (m.lora_A.grad, ref["dA"], "dA"),
                         (m.lora_B.grad, ref["dB"], "dB"), (m.router.gate.weight.grad, ref["dWg"], "dWg")):
        assert got is not None, n
        emax, enorm = _rel(f(got).reshape(want.shape), want)
        print(f"  {n}: max-rel {emax:.2e} norm-rel {enorm:.2e}", flush=True)
        assert emax <= tol and enorm <= tol, f"{n}: max-rel {emax:.3e} norm-rel {enorm:.3e}"
    # torch's ln2 in front of the same layer (autograd through torch's layer_norm)
    grads = [t.grad.clone() for t in (x, ln.weight, ln.bias, m.lora_A)]
    for t in (x, ln.weight, ln.bias, m.lora_A, m.lora_B, m.router.gate.weight):
        t.grad = None
    xn_t = torch.nn.functional.layer_norm(x.float(), (C,), ln.weight.float(), ln.bias.float(), eps=1e-5).to(dt)
    out2, aux2, z2 = m(xn_t, residual=x)
    ((out2.float() * dO.float()).sum() + 0.3 * aux2 - 0.7 * z2).backward()
    for g0, t, n in zip(grads, (x, ln.weight, ln.bias, m.lora_A), ("dx", "d_ln_weight", "d_ln_bias", "dA")):
        emax, enorm = _rel(f(g0), f(t.grad))
        assert emax <= 2 * tol and enorm <= 2 * tol, f"vs torch ln2, {n}: {emax:.3e} {enorm:.3e}"


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_experts_module_block_form_autograd(device, dtype):
    """MoE_CMix(x, x_prev, residual=x, ln=ln2) under autograd against the
    oracle: the full-expert VJP at LN(x), then ln2's VJP plus dO."""
    import torch
    from rwkv_mlx_amd import MoE_CMix, RWKVConfig
    B, T, C, F, E, k = 2, 20, 128, 256, 4, 2
    rng = np.random.default_rng(80)
    r = lambda a: O.round_to(a, dtype)
    g = {"x": r(rng.standard_normal((B, T, C)) * 1.5 + 0.3), "x_k": r(rng.uniform(0, 1, (E, C))),
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
    ln = _ln_module(C, dtype, device, seed=81)
    x = to_dev(g["x"], dtype, device).requires_grad_(True)
    xp = to_dev(g["x_prev"], dtype, device).requires_grad_(True)
    out, aux, z = m(x, x_prev=xp, residual=x, ln=ln)
    ((out.float() * to_dev(g["dO"], dtype, device).float()).sum() + 0.3 * aux - 0.7 * z).backward()
    f = lambda t: t.detach().float().cpu().numpy()
    N = B * T
    w, b = f(ln.weight), f(ln.bias)
    xn = O.layer_norm(g["x"].reshape(N, C), w, b, dtype).reshape(B, T, C)
    p = {"x_k": g["x_k"], "Wk": g["Wk"], "Wv": g["Wv"], "Wg": g["Wg"]}
    ref = MB.experts_backward(xn, p, k, dtype, g["dO"], 0.3, -0.7, x_prev=g["x_prev"])
    lref = MB.layer_norm_backward(g["x"].reshape(N, C), w, O.round_to(np.asarray(ref["dx"]).reshape(N, C), dtype),
                                  d_res=g["dO"].reshape(N, C))
    tol = TOL[dtype] if dtype != "f32" else 1e-4
    for got, want, n in ((x.grad, lref["dx"], "dx"), (ln.weight.grad, lref["dw"], "d_ln_weight"),
                         (ln.bias.grad, lref["db"], "d_ln_bias"), (xp.grad, ref["dx_prev"], "dx_prev"),
                         (m.expert_val.grad, ref["dWv"], "dWv"), (m.router.gate.weight.grad, ref["dWg"], "dWg")):
        assert got is not None, n
        want = np.asarray(want)
        emax, enorm = _rel(f(got).reshape(want.shape), want)
        print(f"  {n}: max-rel {emax:.2e} norm-rel {enorm:.2e}", flush=True)
        assert emax <= tol and enorm <= tol, f"{n}: max-rel {emax:.3e} norm-rel {enorm:.3e}"


def _rel(got, ref):
    from helpers import rel_errs
    assert np.all(np.isfinite(got))
    return rel_errs(got, ref)
