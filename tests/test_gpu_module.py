"""The PyTorch drop-in modules on the GPU against the oracle: LoRAMoE_CMix
(moe.py:93-163), Router (moe.py:35-86) and RWKV_CMix_x070
(model.py:243-263), with the reference's parameter names, MLX dtype
promotion, the decode step, the residual add and empty inputs."""
from __future__ import annotations

import math

import numpy as np
import pytest

from helpers import TOL, assert_close, to_np
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def _module(C=128, F=256, E=4, r=8, k=2, seed=0, dtype=None):
    import torch
    from rwkv_mlx_amd.moe import build_layer
    torch.manual_seed(seed)
    m = build_layer(C, F, E, k, r)
    with torch.no_grad():
        m.base.x_k.uniform_(0, 1)
        m.lora_B.normal_(0, 0.02)  # the reference initialises B to zero; a non-zero B exercises the adapters
    m = m.cuda()
    if dtype is not None:
        m = m.to(dtype)
    return m


def _params(m, dtype):
    """The module's parameters as oracle inputs, rounded to `dtype`."""
    f = lambda t: O.round_to(t.detach().float().cpu().numpy(), dtype)
    return {"x_k": f(m.base.x_k).reshape(-1), "Wk": f(m.base.key.weight), "Wv": f(m.base.value.weight),
            "Wg": f(m.router.gate.weight), "A": f(m.lora_A), "B": f(m.lora_B)}


@pytest.mark.parametrize("name,tdt", [("f16", "float16"), ("bf16", "bfloat16")])
def test_lora_moe_cmix_matches_oracle(name, tdt):
    import torch
    dt = getattr(torch, tdt)
    m = _module(dtype=dt)
    x = torch.randn(2, 33, 128, device="cuda").to(dt)
    extras = {}
    out, aux, z = m(x, extras=extras)
    assert out.dtype == dt and out.shape == x.shape
    p = _params(m, name)
    xr = to_np(x)
    ref_out, ref_aux, ref_z = O.moe_forward(xr, p, 2, name)
    assert_close(to_np(out), ref_out, name, "module out")
    assert math.isclose(float(aux), ref_aux, rel_tol=1e-5)
    assert math.isclose(float(z), ref_z, rel_tol=1e-5)
    r = O.router(xr.reshape(-1, 128), p["Wg"], 2, name)
    assert np.array_equal(extras["inds"].cpu().numpy(), r["inds"])
    # sparse mode gives the same result within tolerance
    out_s, _, _ = m(x, mode="sparse")
    assert_close(to_np(out_s), ref_out, name, "module out (sparse)")


def test_fp32_layer_with_fp16_input_runs_in_fp32():
    """A wholly fp32 layer fed fp16 activations runs in fp32 with an fp32 output
    (MLX promotion of x with fp32 weights).  This build upcasts x first, so
    shift(x) - x is rounded to fp32 where MLX rounds it to fp16: a documented
    deviation for a combination the reference's converter does not produce
    (it writes fp16 or fp32 models).  The reference's fine-tune layer, an fp16
    base with fp32 adapters and gate, is pinned in test_gpu_mixed.py."""
    import torch
    m = _module()  # fp32 parameters
    x = torch.randn(1, 20, 128, device="cuda").half()
    out, aux, z = m(x)
    assert out.dtype == torch.float32
    p = _params(m, "f32")
    ref_out, ref_aux, ref_z = O.moe_forward(to_np(x), p, 2, "f32")
    assert_close(to_np(out), ref_out, "f32", "promoted out")
    assert math.isclose(float(aux), ref_aux, rel_tol=1e-5)
    assert math.isclose(float(z), ref_z, rel_tol=1e-5)


def test_decode_step_equals_two_token_forward():
    import torch
    m = _module(dtype=torch.float16)
    xp = torch.randn(6, 128, device="cuda").half()
    x = torch.randn(6, 128, device="cuda").half()
    out, aux, z, state = m.decode_step(x, xp)
    assert torch.equal(state, x)
    full, _, _ = m(torch.stack([xp, x], dim=1))
    assert_close(to_np(out), to_np(full[:, 1]), "f16", "decode vs forward")
    p = _params(m, "f16")
    ref = O.cmix_decode(to_np(x), to_np(xp), p["x_k"], p["Wk"], p["Wv"], "f16")[0]
    base = to_np(m.base(x.unsqueeze(1), x_prev=xp)).reshape(6, -1)
    assert_close(base, ref, "f16", "decode base")


def test_residual_and_orthogonal_loss():
    import torch
    m = _module(dtype=torch.float16)
    x = torch.randn(2, 16, 128, device="cuda").half()
    res = torch.randn_like(x)
    out, _, _ = m(x)
    out_r, _, _ = m(x, residual=res)
    assert torch.equal(out_r, (res.float() + out.float()).half())
    ortho = m.orthogonal_loss()
    ref = O.ortho_loss(_params(m, "f16")["A"], "f16")
    assert math.isclose(float(ortho), ref, rel_tol=2e-2)


def test_router_module():
    import torch
    from rwkv_mlx_amd.moe import Router
    torch.manual_seed(3)
    rt = Router(128, 6, 3).cuda().half()
    x = torch.randn(2, 9, 128, device="cuda").half()
    with torch.no_grad():
        inds, w, aux, z = rt(x)
    assert inds.dtype == torch.int32 and inds.shape == (2, 9, 3)
    assert w.dtype == torch.float16 and w.shape == (2, 9, 3)
    wg = O.round_to(rt.gate.weight.detach().float().cpu().numpy(), "f16")
    r = O.router(to_np(x).reshape(-1, 128), wg, 3, "f16")
    assert np.array_equal(inds.reshape(-1, 3).cpu().numpy(), r["inds"])
    assert np.max(np.abs(to_np(w).reshape(-1, 3) - r["gates"])) <= 2.0 ** -10
    assert math.isclose(float(aux), r["aux"], rel_tol=1e-5)
    assert math.isclose(float(z), r["z"], rel_tol=1e-5)


def test_cmix_base_module():
    import torch
    m = _module(dtype=torch.bfloat16)
    x = torch.randn(3, 11, 128, device="cuda").to(torch.bfloat16)
    out = m.base(x)
    p = _params(m, "bf16")
    ref = O.cmix_base(to_np(x), p["x_k"], p["Wk"], p["Wv"], "bf16")
    assert_close(to_np(out), ref, "bf16", "base module")


def test_empty_input():
    import torch
    m = _module(dtype=torch.float16)
    x = torch.empty(0, 7, 128, device="cuda").half()
    out, aux, z = m(x)
    assert out.shape == (0, 7, 128)
    assert math.isnan(float(aux)) and math.isnan(float(z))
    inds, w, aux2, z2 = m.router(x)
    assert inds.shape == (0, 7, 2) and math.isnan(float(aux2))
    assert m.base(x).shape == (0, 7, 128)
