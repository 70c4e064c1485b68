"""Pins of the ln2 restatement (oracle/moe_oracle.py ``layer_norm``, the
Block's nn.LayerNorm in front of the ChannelMix, model.py:283, 321, and the
RNN form _layer_norm_1d, model.py:434-438) on the CPU.

* The statistics against torch's float64 mean and variance and the output
  steps against the same fp32 steps in torch: equal in every element; the
  whole against torch.nn.functional.layer_norm in float64 (an independent
  implementation) within one step of the dtype.
* Closed forms: a constant row gives y = b exactly; w = 1, b = 0 gives rows
  of mean 0 and variance var / (var + eps); LN(a·x + c) = LN(x) for a > 0
  up to the eps term.
* The reference's RNN form evaluated step by step in float16 (MLX ops on
  fp16 arrays) stays within the fp16 tolerance of the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_oracle as O


def _row_data(n, C, dtype, seed):
    rng = np.random.default_rng(seed)
    x = O.round_to(rng.standard_normal((n, C)) * 2.0 + 0.5, dtype)
    w = O.round_to(1.0 + 0.2 * rng.standard_normal(C), dtype)
    b = O.round_to(0.1 * rng.standard_normal(C), dtype)
    return x, w, b


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("C", [64, 768, 2048])
def test_matches_torch(dtype, C):
    """The statistics against torch's float64 mean / var, the output steps
    against the same steps in torch float32: equal in every element; and the
    whole against torch's float64 layer_norm within one step of the dtype
    (fp32: 4 ulp) — the fp32 output steps are all that separate them."""
    torch = pytest.importorskip("torch")
    x, w, b = _row_data(33, C, dtype, seed=C)
    got = O.layer_norm(x, w, b, dtype)
    x64 = torch.from_numpy(x.astype(np.float64))
    mean = x64.mean(dim=-1, keepdim=True)
    var = x64.var(dim=-1, unbiased=False, keepdim=True)
    rstd = 1.0 / torch.sqrt(var + 1e-5)
    x32, w32, b32 = (torch.from_numpy(a.astype(np.float32)) for a in (x, w, b))
    y = (x32 - mean.float()) * rstd.float() * w32 + b32
    assert np.array_equal(got, O.round_to(y.numpy(), dtype))
    ref = torch.nn.functional.layer_norm(x64, (C,), torch.from_numpy(w.astype(np.float64)),
                                         torch.from_numpy(b.astype(np.float64)), eps=1e-5).numpy()
    # error scale: the size of the terms y is the sum of (fp32 steps), or of y
    # itself (the final rounding to a 16-bit dtype)
    terms = np.abs(((x64 - mean) * rstd).numpy() * w) + np.abs(b)
    scale = terms if dtype == "f32" else np.maximum(np.abs(ref), 4 * 2.0 ** -23 * terms)
    step = {"f32": 4 * 2.0 ** -23, "f16": 2.0 ** -10, "bf16": 2.0 ** -7}[dtype]
    assert np.all(np.abs(got - ref) <= step * scale + 2.0 ** -24)


def test_constant_row_gives_bias():
    C = 256
    x = np.full((3, C), 1.75, np.float32)
    _, w, b = _row_data(1, C, "f32", seed=3)
    assert np.array_equal(O.layer_norm(x, w, b, "f32"), np.broadcast_to(b, (3, C)))


def test_unit_affine_moments_and_invariance():
    C = 1024
    x, _, _ = _row_data(8, C, "f32", seed=4)
    one, zero = np.ones(C, np.float32), np.zeros(C, np.float32)
    y = O.layer_norm(x, one, zero, "f32").astype(np.float64)
    var = x.astype(np.float64).var(axis=1)
    assert np.max(np.abs(y.mean(axis=1))) < 1e-6
    assert np.allclose(y.var(axis=1), var / (var + 1e-5), rtol=1e-5, atol=0)
    y2 = O.layer_norm(3.0 * x.astype(np.float64) - 7.0, one, zero, "f32")
    assert np.max(np.abs(y2 - y)) < 2e-5


def test_rnn_form_in_fp16_within_tolerance():
    """_layer_norm_1d on an fp16 row, each op in fp16 (model.py:434-438)."""
    C = 768
    x, w, b = _row_data(16, C, "f16", seed=5)
    x16, w16, b16 = x.astype(np.float16), w.astype(np.float16), b.astype(np.float16)
    for i in range(x.shape[0]):
        r = x16[i]
        mean = r.mean(dtype=np.float32).astype(np.float16)
        d = (r - mean).astype(np.float16)
        var = (d * d).astype(np.float16).mean(dtype=np.float32).astype(np.float16)
        y = (d / np.sqrt(var + np.float16(1e-5)).astype(np.float16)).astype(np.float16) * w16 + b16
        ref = O.layer_norm(x[i:i + 1], w, b, "f16")[0]
        err = np.max(np.abs(y.astype(np.float64) - ref)) / np.max(np.abs(ref))
        assert err <= 2e-2, err


# ---- the VJP (oracle/moe_backward.layer_norm_backward) ----------------------------------

def _ln64(x, w, b, eps=1e-5):
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * w + b


@pytest.mark.parametrize("C", [64, 768, 2048])
def test_backward_matches_torch_autograd(C):
    """Against torch autograd of layer_norm in float64 (an independent
    implementation of the same derivative): within 1e-12 relative."""
    torch = pytest.importorskip("torch")
    from oracle import moe_backward as MB
    rng = np.random.default_rng(C + 1)
    x, w, b = _row_data(40, C, "f32", seed=C + 2)
    dy = rng.standard_normal(x.shape)
    xt = torch.from_numpy(x.astype(np.float64)).requires_grad_(True)
    wt = torch.from_numpy(w.astype(np.float64)).requires_grad_(True)
    bt = torch.from_numpy(b.astype(np.float64)).requires_grad_(True)
    torch.nn.functional.layer_norm(xt, (C,), wt, bt, eps=1e-5).backward(torch.from_numpy(dy))
    got = MB.layer_norm_backward(x, w, dy)
    for name, ref in (("dx", xt.grad), ("dw", wt.grad), ("db", bt.grad)):
        ref = ref.numpy()
        assert np.max(np.abs(got[name] - ref)) <= 1e-12 * np.max(np.abs(ref)), name


def test_backward_central_differences():
    """<dy, LN(x)> differentiated numerically in x, w and b (float64)."""
    from oracle import moe_backward as MB
    rng = np.random.default_rng(7)
    C = 64
    x, w, b = [a.astype(np.float64) for a in _row_data(3, C, "f32", seed=8)]
    dy = rng.standard_normal(x.shape)
    d_res = rng.standard_normal(x.shape)
    got = MB.layer_norm_backward(x, w, dy, d_res=d_res)
    f = lambda xx, ww, bb: float((dy * _ln64(xx, ww, bb)).sum() + (d_res * xx).sum())
    h = 1e-6
    for (i, j) in [(0, 0), (1, 17), (2, 63)]:
        e = np.zeros_like(x)
        e[i, j] = h
        num = (f(x + e, w, b) - f(x - e, w, b)) / (2 * h)
        assert abs(num - got["dx"][i, j]) <= 1e-6 * max(1.0, abs(num))
    for j in (0, 31, 63):
        e = np.zeros(C)
        e[j] = h
        assert abs((f(x, w + e, b) - f(x, w - e, b)) / (2 * h) - got["dw"][j]) <= 1e-6
        assert abs((f(x, w, b + e) - f(x, w, b - e)) / (2 * h) - got["db"][j]) <= 1e-6


def test_backward_invariants_and_planted_mistake():
    """LN(x) is unchanged by x → x + c and (to the eps term) by x → a·x, so
    dx is orthogonal to 1 in every row and, with eps = 0, to x̂ (with eps the
    closed form below); dy constant along a row
    with w = 1 gives dx = 0.  Dropping the x̂·mean(g⊙x̂) term (a plausible
    mistake, planted here) breaks the second invariant."""
    from oracle import moe_backward as MB
    rng = np.random.default_rng(9)
    C = 768
    x, w, _ = [a.astype(np.float64) for a in _row_data(16, C, "f32", seed=10)]
    dy = rng.standard_normal(x.shape)
    mean = x.mean(axis=1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=1, keepdims=True)
    g = dy * w
    for eps in (0.0, 1e-5):
        dx = MB.layer_norm_backward(x, w, dy, eps=eps)["dx"]
        xh = (x - mean) / np.sqrt(var + eps)
        scale = np.abs(dx).max()
        assert np.max(np.abs(dx.sum(axis=1))) <= 1e-10 * scale * C
        # Σ dx·x̂ = rstd · eps / (var + eps) · Σ g·x̂ (0 without the eps term)
        want = (g * xh).sum(axis=1) * eps / (var[:, 0] + eps) / np.sqrt(var[:, 0] + eps)
        assert np.max(np.abs((dx * xh).sum(axis=1) - want)) <= 1e-10 * scale * C
    const = np.repeat(rng.standard_normal((16, 1)), C, axis=1)
    assert np.max(np.abs(MB.layer_norm_backward(x, np.ones(C), const)["dx"])) <= 1e-12
    rstd = 1.0 / np.sqrt(var + 1e-5)
    bad = rstd * (g - g.mean(axis=1, keepdims=True))
    assert np.max(np.abs((bad * xh).sum(axis=1))) > 1e-2 * scale * C
