"""GPU parity of the backward (rwkvmoe_backward, through the C ABI) against
the float64 backward oracle (oracle/moe_backward.py, itself pinned by finite
differences), and of the torch autograd path of LoRAMoE_CMix.

Each case runs the forward (for the logits and selection it saves), then the
backward with a seeded d_out and non-zero aux / z cotangents, and checks
d_x, d_lora_A, d_lora_B and d_w_gate.  Tolerance (max|got-ref| / max|ref|
and the 2-norm ratio): 1e-5 for fp32 layers, 2e-2 for fp16 / bf16 (the
intermediate products are rounded to the layer dtype, as MLX's fp16 / bf16
VJPs round them).  Also: the backward run twice is bit-identical; outputs
left NULL change nothing else; with lora_B = 0, d_lora_A is exactly zero.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import Layer, to_np
from oracle import moe_backward as MB
from rwkv_mlx_amd.workloads import LayerShape, make_inputs

pytestmark = pytest.mark.gpu

BWD_TOL = {"f32": 1e-5, "f16": 2e-2, "bf16": 2e-2}
D_LOSSES = (0.3, -0.7)

CASES = {
    "bwd-c128-e4-k2-r8-f32": LayerShape("bwd-c128-e4-k2-r8-f32", "f32", 2, 24, 128, 256, 4, 2, 8, seed=8001),
    "bwd-c128-e4-k2-r8-f16": LayerShape("bwd-c128-e4-k2-r8-f16", "f16", 2, 24, 128, 256, 4, 2, 8, seed=8002),
    "bwd-c128-e4-k2-r8-bf16": LayerShape("bwd-c128-e4-k2-r8-bf16", "bf16", 2, 24, 128, 256, 4, 2, 8, seed=8003),
    "bwd-ragged-e5-k3-r3-f16": LayerShape("bwd-ragged-e5-k3-r3-f16", "f16", 3, 37, 128, 256, 5, 3, 3, seed=8004),
    "bwd-e1-k1-r4-bf16": LayerShape("bwd-e1-k1-r4-bf16", "bf16", 1, 40, 64, 128, 1, 1, 4, seed=8005),
    "bwd-d768-e8-k2-r16-f16": LayerShape("bwd-d768-e8-k2-r16-f16", "f16", 1, 512, 768, 3072, 8, 2, 16, seed=8006),
    "bwd-e64-k8-r32-f16": LayerShape("bwd-e64-k8-r32-f16", "f16", 2, 40, 192, 320, 64, 8, 32, seed=8007),
    "bwd-skew-e32-k4-f32": LayerShape("bwd-skew-e32-k4-f32", "f32", 1, 96, 256, 512, 32, 4, 16, zipf_s=1.2,
                                      seed=8008),
    "bwd-decode-e8-k2-bf16": LayerShape("bwd-decode-e8-k2-bf16", "bf16", 64, 1, 768, 3072, 8, 2, 16, decode=True,
                                        seed=8009),
    # fused routing kernel with Kx = 128 and padding columns (E·r = 96), C = 256, ragged tokens
    "bwd-c256-e6-k2-r16-f16": LayerShape("bwd-c256-e6-k2-r16-f16", "f16", 3, 67, 256, 512, 6, 2, 16, seed=8010),
    # fused routing kernel, top-1, C = 512, bf16
    "bwd-c512-e8-k1-r16-bf16": LayerShape("bwd-c512-e8-k1-r16-bf16", "bf16", 2, 99, 512, 1024, 8, 1, 16, seed=8011),
    # 16-bit layer beyond the fused kernel (Kx = 512) with a Zipf bias: the
    # hot expert's ranges hold several 128-token chunks for the per-expert
    # contractions
    "bwd-skew-e32-k4-f16": LayerShape("bwd-skew-e32-k4-f16", "f16", 4, 256, 256, 512, 32, 4, 16, zipf_s=1.2,
                                      seed=8012),
    # fp32 layers: an odd rank over ragged tokens, and the limits E = 64,
    # top-8, r = 32
    "bwd-ragged-e5-k3-r3-f32": LayerShape("bwd-ragged-e5-k3-r3-f32", "f32", 3, 37, 128, 256, 5, 3, 3, seed=8013),
    "bwd-e64-k8-r32-f32": LayerShape("bwd-e64-k8-r32-f32", "f32", 2, 200, 192, 320, 64, 8, 32, seed=8014),
}


def _errs(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    mx = max(float(np.max(np.abs(ref))), 1e-30)
    nrm = max(float(np.linalg.norm(ref)), 1e-30)
    return float(np.max(np.abs(got - ref))) / mx, float(np.linalg.norm(got - ref)) / nrm


def _bits(t):
    """The tensor's bytes (exact comparison for every dtype, bf16 included)."""
    return t.detach().contiguous().view(-1).view(__import__("torch").uint8).cpu().numpy()


def _run_backward(L, dO, d_losses, outputs=("d_x", "d_lora_A", "d_lora_B", "d_w_gate"), ex=None):
    import torch
    from rwkv_mlx_amd import _lib
    w = L.w
    if ex is None:
        _, _, ex = L.forward(extras=True)
    shapes = {"d_x": (L.N, w.d_model), "d_lora_A": (w.n_experts, w.d_model, w.lora_rank),
              "d_lora_B": (w.n_experts, w.lora_rank, w.d_model), "d_w_gate": (w.n_experts, w.d_model)}
    outs = {n: torch.full(shapes[n], float("nan"), dtype=L.dt, device=L.dev) for n in outputs}
    nbytes = _lib.backward_workspace_bytes(L.desc)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=L.dev)
    _lib.backward(L.desc, ws, nbytes, _lib.current_stream(L.dev), x=L.x, w_gate=L.Wg, lora_A=L.A, lora_B=L.B,
                  logits=ex["logits"], inds=ex["inds"], d_out=dO, d_losses=d_losses, **outs)
    torch.cuda.synchronize()
    return outs, ex


def _cotangents(L, seed=99):
    import torch
    from helpers import to_dev
    from oracle import moe_oracle as O
    rng = np.random.default_rng(seed)
    dO = O.round_to(rng.standard_normal((L.N, L.w.d_model)), L.w.dtype)
    return dO, to_dev(dO, L.w.dtype, L.dev), torch.tensor(D_LOSSES, dtype=torch.float32, device=L.dev)


@pytest.fixture(scope="module", params=list(CASES))
def case(request, device):
    print(f"\n[backward case] {request.param}", flush=True)
    shape = CASES[request.param]
    L = Layer(shape, device)
    g = L.np
    dO_np, dO, dl = _cotangents(L)
    ref = MB.moe_backward(g["x"].reshape(L.N, -1), g["Wg"], g["A"], g["B"], shape.top_k, shape.dtype, dO_np,
                          D_LOSSES[0], D_LOSSES[1], g.get("bias"))
    return L, dO, dl, ref


def test_backward_matches_oracle(case):
    L, dO, dl, ref = case
    outs, ex = _run_backward(L, dO, dl)
    assert np.array_equal(ex["inds"].cpu().numpy(), ref["inds"])
    tol = BWD_TOL[L.w.dtype]
    w = L.w
    for name, key, shape in (("d_x", "dx", (L.N, w.d_model)), ("d_lora_A", "dA", None), ("d_lora_B", "dB", None),
                             ("d_w_gate", "dWg", None)):
        got = to_np(outs[name])
        want = ref[key].reshape(got.shape)
        assert np.all(np.isfinite(got)), name
        emax, enorm = _errs(got, want)
        print(f"  {name}: max-rel {emax:.2e} norm-rel {enorm:.2e}")
        assert emax <= tol and enorm <= tol, f"{w.name} {name}: max-rel {emax:.3e} norm-rel {enorm:.3e} > {tol}"


def test_backward_is_deterministic_and_outputs_independent(case):
    L, dO, dl, _ = case
    a, ex = _run_backward(L, dO, dl)
    b, _ = _run_backward(L, dO, dl, ex=ex)
    for n in a:
        assert np.array_equal(_bits(a[n]), _bits(b[n])), n
    only_x, _ = _run_backward(L, dO, dl, outputs=("d_x",), ex=ex)
    assert np.array_equal(_bits(only_x["d_x"]), _bits(a["d_x"]))
    only_b, _ = _run_backward(L, dO, dl, outputs=("d_lora_B", "d_w_gate"), ex=ex)
    assert np.array_equal(_bits(only_b["d_lora_B"]), _bits(a["d_lora_B"]))
    assert np.array_equal(_bits(only_b["d_w_gate"]), _bits(a["d_w_gate"]))


def test_zero_lora_B_gives_zero_d_lora_A(device):
    shape = CASES["bwd-c128-e4-k2-r8-f16"]
    g = make_inputs(shape)
    g["B"] = np.zeros_like(g["B"])
    L = Layer(shape, device, inputs=g)
    _, dO, dl = _cotangents(L)
    outs, _ = _run_backward(L, dO, dl)
    assert np.all(to_np(outs["d_lora_A"]) == 0)
    assert np.any(to_np(outs["d_lora_B"]) != 0)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_module_autograd_matches_oracle(device, dtype):
    """LoRAMoE_CMix under torch autograd: loss = <dO, out> + 0.3·aux − 0.7·z,
    gradients of x, lora_A, lora_B, router.gate.weight against the oracle;
    the frozen base receives none."""
    import torch
    from helpers import torch_dtype
    from oracle import moe_oracle as O
    from rwkv_mlx_amd.moe import build_layer
    C, F, E, k, r, B, T = 128, 256, 4, 2, 8, 2, 16
    torch.manual_seed(3)
    m = build_layer(C, F, E, k, r)
    with torch.no_grad():
        m.base.x_k.uniform_(0, 1)
        m.lora_B.normal_(0, 0.05)
    m = m.to(device=device, dtype=torch_dtype(dtype))
    x = torch.randn(B, T, C, generator=torch.Generator().manual_seed(4)).to(device=device, dtype=torch_dtype(dtype))
    x.requires_grad_(True)
    dO = torch.randn(B, T, C, generator=torch.Generator().manual_seed(5)).to(device=device, dtype=torch_dtype(dtype))
    out, aux, z = m(x)
    loss = (out.float() * dO.float()).sum() + 0.3 * aux - 0.7 * z
    loss.backward()
    f = lambda t: t.detach().float().cpu().numpy()
    ref = MB.moe_backward(f(x).reshape(B * T, C), f(m.router.gate.weight), f(m.lora_A), f(m.lora_B), k, dtype,
                          O.round_to(f(dO).reshape(B * T, C), dtype), 0.3, -0.7)
    tol = BWD_TOL[dtype]
    for got, key in ((x.grad, "dx"), (m.lora_A.grad, "dA"), (m.lora_B.grad, "dB"), (m.router.gate.weight.grad, "dWg")):
        assert got is not None, key
        emax, enorm = _errs(f(got).reshape(ref[key].shape), ref[key])
        assert emax <= tol and enorm <= tol, f"{key}: {emax:.3e} {enorm:.3e}"
    assert m.base.key.weight.grad is None and m.base.value.weight.grad is None and m.base.x_k.grad is None


@pytest.mark.parametrize("dtype,E,C,r", [("f32", 4, 128, 8), ("f16", 8, 768, 16), ("bf16", 5, 192, 3),
                                         ("f16", 64, 256, 32)])
def test_ortho_backward_matches_oracle(device, dtype, E, C, r):
    """rwkvmoe_ortho_backward against the float64 gradient of
    orthogonal_loss, scaled by a cotangent, through the C ABI and through
    autograd (LoRAMoE_CMix.orthogonal_loss().backward())."""
    import torch
    from helpers import to_dev, torch_dtype
    from oracle import moe_oracle as O
    from rwkv_mlx_amd import _lib
    from rwkv_mlx_amd.moe import build_layer
    rng = np.random.default_rng(E * 1000 + C)
    A_np = O.round_to(rng.standard_normal((E, C, r)) / np.sqrt(C), dtype)
    d = 0.37
    ref = d * MB.ortho_grad(A_np)
    A = to_dev(A_np, dtype, device)
    dA = torch.full_like(A, float("nan"))
    desc = _lib.make_desc(1, 1, C, 64, E, 1, r, dtype)
    nbytes = _lib.backward_workspace_bytes(desc)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    dl = torch.tensor([d], dtype=torch.float32, device=device)
    _lib.backward(desc, ws, nbytes, _lib.current_stream(device), entry="rwkvmoe_ortho_backward", lora_A=A,
                  d_lora_A=dA, d_ortho=dl)
    torch.cuda.synchronize()
    tol = BWD_TOL[dtype]
    emax, enorm = _errs(to_np(dA), ref)
    assert emax <= tol and enorm <= tol, f"{emax:.3e} {enorm:.3e}"
    # autograd
    m = build_layer(C, 128, E, 1, r).to(device=device, dtype=torch_dtype(dtype))
    with torch.no_grad():
        m.lora_A.copy_(A)
    loss = m.orthogonal_loss() * d
    loss.backward()
    emax, enorm = _errs(to_np(m.lora_A.grad), ref)
    assert emax <= tol and enorm <= tol, f"autograd {emax:.3e} {enorm:.3e}"
