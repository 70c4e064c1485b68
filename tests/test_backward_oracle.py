"""Pins of the backward oracle (oracle/moe_backward.py) on the CPU.

* Every gradient entry against central finite differences of the float64
  forward ``smooth_loss`` (selection and counts held at their values at the
  point), for top-1/2/3, with a logit bias and non-zero aux / z cotangents.
* ``smooth_loss``'s delta, aux and z against the pinned forward oracle
  (moe_oracle.moe_forward) at fp32.
* Closed forms: B = 0 gives dA = 0 and a dx with only the router terms;
  with zero loss cotangents and one expert (k = 1) the gates are 1 and the
  router receives no gradient from the output.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_backward as MB
from oracle import moe_oracle as O


def _case(N, C, E, r, k, seed, bias=False):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((N, C)).astype(np.float32)
    Wg = (rng.standard_normal((E, C)) / np.sqrt(C)).astype(np.float32)
    A = (rng.standard_normal((E, C, r)) / np.sqrt(C)).astype(np.float32)
    B = (rng.standard_normal((E, r, C)) * 0.3).astype(np.float32)
    dO = rng.standard_normal((N, C)).astype(np.float32)
    b = (rng.standard_normal(E) * 0.5).astype(np.float32) if bias else None
    return x, Wg, A, B, dO, b


@pytest.mark.parametrize("k,bias,d_aux,d_z", [(1, False, 0.0, 0.0), (2, False, 0.7, -1.3), (3, True, 2.0, 0.5),
                                              (2, True, 0.0, 3.0)])
def test_gradients_match_finite_differences(k, bias, d_aux, d_z):
    N, C, E, r = 7, 64, 4, 3
    x, Wg, A, B, dO, b = _case(N, C, E, r, k, seed=11 + k, bias=bias)
    g = MB.moe_backward(x, Wg, A, B, k, "f32", dO, d_aux, d_z, b)
    rt = O.router(x, Wg, k, "f32", b)
    inds, counts = rt["inds"], rt["counts"]
    x64, Wg64, A64, B64 = (v.astype(np.float64) for v in (x, Wg, A, B))

    def L(xx, ww, aa, bb):
        return MB.smooth_loss(xx, ww, aa, bb, inds, counts, dO, d_aux, d_z, b)[0]

    eps = 1e-6
    pick = np.random.default_rng(k)
    for name, arr, idx in (("dx", x64, 0), ("dWg", Wg64, 1), ("dA", A64, 2), ("dB", B64, 3)):
        # 80 entries of each gradient, drawn at random
        flat = pick.choice(arr.size, size=min(80, arr.size), replace=False)
        fd = np.zeros(flat.size)
        for n, f in enumerate(flat):
            i = np.unravel_index(f, arr.shape)
            args = [x64, Wg64, A64, B64]
            hi = [a.copy() for a in args]
            lo = [a.copy() for a in args]
            hi[idx][i] += eps
            lo[idx][i] -= eps
            fd[n] = (L(*hi) - L(*lo)) / (2 * eps)
        got = g[name].reshape(-1)[flat]
        scale = np.max(np.abs(g[name])) + 1e-12
        err = np.max(np.abs(got - fd)) / scale
        assert err < 2e-5, f"{name}: max rel err {err:.3g}"
    # the selection did not move under the perturbations (no near-ties)
    lg = rt["logits"].astype(np.float64)
    srt = np.sort(lg, axis=1)[:, ::-1]
    if k < E:
        assert np.min(srt[:, k - 1] - srt[:, k]) > 1e-4


def test_smooth_loss_matches_forward_oracle():
    N, C, E, r, k = 9, 64, 5, 4, 2
    x, Wg, A, B, dO, b = _case(N, C, E, r, k, seed=3, bias=True)
    parts = O.moe_forward(x.reshape(1, N, C), {"x_k": np.zeros(C, np.float32), "Wk": np.zeros((64, C), np.float32),
                                               "Wv": np.zeros((C, 64), np.float32), "Wg": Wg, "A": A, "B": B},
                          k, "f32", bias=b, return_parts=True)
    _, delta, aux, z = MB.smooth_loss(x, Wg, A, B, parts["inds"], parts["counts"], dO, bias=b)
    assert np.max(np.abs(delta - parts["delta"])) <= 1e-5 * np.max(np.abs(delta))
    assert abs(aux - parts["aux"]) <= 1e-5 * abs(aux)
    assert abs(z - parts["z"]) <= 1e-5 * abs(z)


def test_zero_B_closed_form():
    N, C, E, r, k = 6, 64, 3, 2, 2
    x, Wg, A, B, dO, _ = _case(N, C, E, r, k, seed=5)
    B[:] = 0
    g = MB.moe_backward(x, Wg, A, B, k, "f32", dO, 0.4, 0.9)
    assert np.all(g["dA"] == 0)
    assert np.all(g["dg"] == 0)  # a_e = 0
    # dx is the router term alone: dℓ·W_gate
    assert np.allclose(g["dx"], g["dlogits"] @ Wg.astype(np.float64), rtol=0, atol=1e-12)
    # dB_e = s_eᵀ (w_e ⊙ dO) is unaffected by B
    rt = O.router(x, Wg, k, "f32")
    w = O.gate_dense(rt["inds"], rt["gates"], E).astype(np.float64)
    for e in range(E):
        s_e = O._mm(x, A[e], "f32").astype(np.float64)
        assert np.allclose(g["dB"][e], s_e.T @ (w[:, e:e + 1] * dO), rtol=1e-12, atol=1e-12)


def test_single_expert_gates_are_constant():
    N, C, E, r, k = 5, 64, 1, 2, 1
    x, Wg, A, B, dO, _ = _case(N, C, E, r, k, seed=9)
    g = MB.moe_backward(x, Wg, A, B, k, "f32", dO, 0.0, 0.0)
    assert np.all(g["dlogits"] == 0) and np.all(g["dWg"] == 0)
    # δ = (x A) B exactly with gate 1: dx = dO Bᵀ Aᵀ
    want = dO.astype(np.float64) @ B[0].astype(np.float64).T @ A[0].astype(np.float64).T
    assert np.allclose(g["dx"], want, rtol=1e-12, atol=1e-12)


def test_ortho_grad_matches_finite_differences_and_closed_forms():
    rng = np.random.default_rng(21)
    E, C, r = 4, 64, 3
    A = rng.standard_normal((E, C, r))
    g = MB.ortho_grad(A)
    eps = 1e-6
    for f in rng.choice(A.size, size=80, replace=False):
        i = np.unravel_index(f, A.shape)
        hi, lo = A.copy(), A.copy()
        hi[i] += eps
        lo[i] -= eps
        fd = (MB.ortho_loss64(hi) - MB.ortho_loss64(lo)) / (2 * eps)
        assert abs(g[i] - fd) <= 2e-5 * np.max(np.abs(g))
    # the float64 loss is the oracle's at fp32 up to rounding
    assert abs(MB.ortho_loss64(A.astype(np.float32)) - O.ortho_loss(A.astype(np.float32), "f32")) \
        <= 1e-5 * MB.ortho_loss64(A)
    # mutually orthogonal column spaces: loss 0 and gradient 0
    Q, _ = np.linalg.qr(rng.standard_normal((C, E * r)))
    Ao = np.stack([Q[:, e * r:(e + 1) * r] for e in range(E)])
    assert np.max(np.abs(MB.ortho_grad(Ao))) < 1e-12
    # Euler: the loss is homogeneous of degree 4, so <A, dA> = 4 loss
    assert abs(np.sum(A * g) - 4 * MB.ortho_loss64(A)) <= 1e-9 * abs(4 * MB.ortho_loss64(A))


def test_fine_tune_layer_mode():
    """The fine-tune layer (fp16 x, fp32 gate and adapters; moe.py:47, 56, 86,
    124-125): the router cotangents equal the all-fp32 ones (same logits, and
    s_e, a_e in fp32 in both), and dA / dB are the finite differences of the
    output with the gates held at their fp16-rounded values (moe.py:86)."""
    N, C, E, r, k = 6, 64, 4, 3, 2
    x, Wg, A, B, dO, _ = _case(N, C, E, r, k, seed=21)
    x = O.round_to(x, "f16")
    g = MB.moe_backward(x, Wg, A, B, k, "f16", dO, 0.4, -0.6, gate_dtype="f32", adapter_dtype="f32")
    g32 = MB.moe_backward(x, Wg, A, B, k, "f32", dO, 0.4, -0.6)
    assert np.array_equal(g["dlogits"], g32["dlogits"]) and np.array_equal(g["dWg"], g32["dWg"])
    rt = O.router(x, Wg, k, "f16", gate_dtype="f32")
    w = O.gate_dense(rt["inds"], rt["gates"], E).astype(np.float64)  # fp16-rounded gates
    assert not np.array_equal(w, O.gate_dense(rt["inds"], O.router(x, Wg, k, "f32")["gates"], E))
    x64, d64 = x.astype(np.float64), dO.astype(np.float64)

    def L(aa, bb):
        return float(np.sum(d64 * sum(w[:, e:e + 1] * ((x64 @ aa[e]) @ bb[e]) for e in range(E))))

    eps = 1e-6
    A64, B64 = A.astype(np.float64), B.astype(np.float64)
    for name, idx in (("dA", 0), ("dB", 1)):
        arr = (A64, B64)[idx]
        flat = np.random.default_rng(idx).choice(arr.size, size=40, replace=False)
        fd = []
        for f in flat:
            i = np.unravel_index(f, arr.shape)
            hi = [A64.copy(), B64.copy()]
            lo = [A64.copy(), B64.copy()]
            hi[idx][i] += eps
            lo[idx][i] -= eps
            fd.append((L(*hi) - L(*lo)) / (2 * eps))
        got = g[name].reshape(-1)[flat]
        err = np.max(np.abs(got - np.array(fd))) / (np.max(np.abs(g[name])) + 1e-12)
        assert err < 2e-6, f"{name}: {err:.3g}"


# ---- the standalone Router's VJP (router_backward) --------------------------------

@pytest.mark.parametrize("k,bias,d_aux,d_z", [(1, False, 0.0, 0.0), (2, False, 0.7, -1.3), (3, True, 2.0, 0.5),
                                              (2, True, 0.0, 3.0)])
def test_router_gradients_match_finite_differences(k, bias, d_aux, d_z):
    """router_backward against central differences of router_smooth_loss
    (selection and counts held), every entry of dx and dW_gate."""
    N, C, E = 9, 64, 5
    rng = np.random.default_rng(40 + k)
    x = rng.standard_normal((N, C)).astype(np.float32)
    Wg = (rng.standard_normal((E, C)) / np.sqrt(C)).astype(np.float32)
    b = (rng.standard_normal(E) * 0.5).astype(np.float32) if bias else None
    dg = rng.standard_normal((N, k))
    g = MB.router_backward(x, Wg, k, "f32", dg, d_aux, d_z, b)
    rt = O.router(x, Wg, k, "f32", b)
    inds, counts = rt["inds"], rt["counts"]
    x64, Wg64 = x.astype(np.float64), Wg.astype(np.float64)
    eps = 1e-6
    for name, arr, idx in (("dx", x64, 0), ("dWg", Wg64, 1)):
        fd = np.zeros(arr.size)
        for f in range(arr.size):
            i = np.unravel_index(f, arr.shape)
            hi = [x64.copy(), Wg64.copy()]
            lo = [x64.copy(), Wg64.copy()]
            hi[idx][i] += eps
            lo[idx][i] -= eps
            fd[f] = (MB.router_smooth_loss(*hi, inds, counts, dg, d_aux, d_z, b)
                     - MB.router_smooth_loss(*lo, inds, counts, dg, d_aux, d_z, b)) / (2 * eps)
        got = g[name].reshape(-1)
        scale = np.max(np.abs(got)) + 1e-12
        assert np.max(np.abs(got - fd)) <= 1e-6 * max(scale, 1.0), name


def test_router_gradient_is_the_layer_gradients_routing_part():
    """The layer's VJP routes its slot cotangents dg through the same logit
    gradient: router_backward given the layer's dg returns the layer's dℓ
    and its dW_gate (no other path reaches W_gate)."""
    x, Wg, A, B, dO, b = _case(11, 64, 4, 3, 2, seed=77, bias=True)
    lay = MB.moe_backward(x, Wg, A, B, 2, "f32", dO, 0.4, 0.9, b)
    rt = MB.router_backward(x, Wg, 2, "f32", lay["dg"], 0.4, 0.9, b)
    assert np.allclose(rt["dlogits"], lay["dlogits"], rtol=0, atol=1e-12)
    assert np.allclose(rt["dWg"], lay["dWg"], rtol=0, atol=1e-12)


def test_router_closed_forms():
    """Zero cotangents give zero gradients; with k = E the gates are the
    full softmax, whose gradient with an all-ones d_gates is zero (Σ g = 1)."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 64)).astype(np.float32)
    Wg = (rng.standard_normal((3, 64)) / 8).astype(np.float32)
    z = MB.router_backward(x, Wg, 2, "f32", np.zeros((6, 2)))
    assert np.all(z["dx"] == 0) and np.all(z["dWg"] == 0)
    ones = MB.router_backward(x, Wg, 3, "f32", np.ones((6, 3)))
    assert np.max(np.abs(ones["dlogits"])) < 1e-12
