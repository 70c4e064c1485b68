"""Pins of the full-expert (MoE_CMix) backward oracle
(oracle/moe_backward.py ``experts_backward``) on the CPU.

* Every gradient (x, the carried state, x_k, expert_key, expert_val,
  router.gate.weight) against central finite differences of the float64
  forward ``experts_smooth_loss`` (selection and counts held at their values
  at the point), top-1 and top-2, with a logit bias and non-zero aux / z
  cotangents.
* The same gradients, in full, against torch autograd through
  ``experts_smooth_loss`` restated in torch float64 (an independent
  derivative of the same forward).
* ``experts_smooth_loss``'s output, aux and z against the pinned forward
  oracle (moe_oracle.experts_forward) at fp32.
* Closed forms: expert_val = 0 gives no gradient to x_k and expert_key and
  no output term in the router; one expert at top-1 is the plain ChannelMix,
  whose gradient with respect to expert_val is hᵀ·dO.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_backward as MB
from oracle import moe_oracle as O


def _case(Bsz, T, C, F, E, seed, bias=False, prev=True):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((Bsz, T, C)).astype(np.float32)
    p = {"x_k": rng.uniform(0, 1, (E, C)).astype(np.float32),
         "Wk": (rng.standard_normal((E, F, C)) / np.sqrt(C)).astype(np.float32),
         "Wv": (rng.standard_normal((E, C, F)) / np.sqrt(F)).astype(np.float32),
         "Wg": (rng.standard_normal((E, C)) / np.sqrt(C)).astype(np.float32)}
    dO = rng.standard_normal((Bsz, T, C)).astype(np.float32)
    xp = rng.standard_normal((Bsz, C)).astype(np.float32) if prev else None
    b = (rng.standard_normal(E) * 0.5).astype(np.float32) if bias else None
    return x, p, dO, xp, b


@pytest.mark.parametrize("k,bias,d_aux,d_z,prev", [(1, False, 0.0, 0.0, False), (2, True, 0.7, -1.3, True),
                                                   (2, False, 2.0, 0.5, True)])
def test_gradients_match_finite_differences(k, bias, d_aux, d_z, prev):
    Bsz, T, C, F, E = 2, 3, 64, 64, 3
    x, p, dO, xp, b = _case(Bsz, T, C, F, E, seed=31 + k, bias=bias, prev=prev)
    g = MB.experts_backward(x, p, k, "f32", dO, d_aux, d_z, x_prev=xp, bias=b)
    rt = O.router(x.reshape(-1, C), p["Wg"], k, "f32", b)
    inds, counts = rt["inds"], rt["counts"]
    base = {n: np.asarray(v, np.float64) for n, v in p.items()}
    x64 = x.astype(np.float64)
    xp64 = None if xp is None else xp.astype(np.float64)

    def L(xx, pp, xpp):
        return MB.experts_smooth_loss(xx, pp, inds, counts, dO, d_aux, d_z, x_prev=xpp, bias=b)[0]

    eps = 1e-6
    pick = np.random.default_rng(k)
    targets = [("dx", "x"), ("dx_k", "x_k"), ("dWk", "Wk"), ("dWv", "Wv"), ("dWg", "Wg")]
    if xp is not None:
        targets.append(("dx_prev", "x_prev"))
    for gname, what in targets:
        arr = x64 if what == "x" else (xp64 if what == "x_prev" else base[what])
        flat = pick.choice(arr.size, size=min(60, arr.size), replace=False)
        fd = np.zeros(flat.size)
        for n, f in enumerate(flat):
            i = np.unravel_index(f, arr.shape)
            vals = []
            for sgn in (1, -1):
                xx, pp, xpp = x64.copy(), {m: v.copy() for m, v in base.items()}, None if xp64 is None else xp64.copy()
                tgt = xx if what == "x" else (xpp if what == "x_prev" else pp[what])
                tgt[i] += sgn * eps
                vals.append(L(xx, pp, xpp))
            fd[n] = (vals[0] - vals[1]) / (2 * eps)
        got = np.asarray(g[gname]).reshape(-1)[flat]
        scale = np.max(np.abs(g[gname])) + 1e-12
        err = np.max(np.abs(got - fd)) / scale
        assert err < 2e-5, f"{gname}: max rel err {err:.3g}"
    lg = rt["logits"].astype(np.float64)
    srt = np.sort(lg, axis=1)[:, ::-1]
    if k < E:
        assert np.min(srt[:, k - 1] - srt[:, k]) > 1e-4


def test_gradients_match_torch_autograd():
    torch = pytest.importorskip("torch")
    Bsz, T, C, F, E, k = 2, 4, 64, 128, 4, 2
    x, p, dO, xp, b = _case(Bsz, T, C, F, E, seed=41, bias=True)
    d_aux, d_z = 0.3, -0.8
    g = MB.experts_backward(x, p, k, "f32", dO, d_aux, d_z, x_prev=xp, bias=b)
    rt = O.router(x.reshape(-1, C), p["Wg"], k, "f32", b)
    inds = torch.from_numpy(rt["inds"].astype(np.int64))
    f = torch.from_numpy(rt["counts"].astype(np.float64)) / (Bsz * T * k)
    tx = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    txp = torch.tensor(xp, dtype=torch.float64, requires_grad=True)
    tp = {n: torch.tensor(v, dtype=torch.float64, requires_grad=True) for n, v in p.items()}
    flat = tx.reshape(-1, C)
    lg = flat @ tp["Wg"].T + torch.tensor(b, dtype=torch.float64)
    g_sel = torch.softmax(torch.gather(lg, 1, inds), dim=-1)
    prev = torch.cat([txp[:, None, :], tx[:, :-1]], dim=1)
    xx = (prev - tx).reshape(-1, C)
    out = torch.zeros_like(flat)
    for e in range(E):
        he = torch.relu((flat + xx * tp["x_k"][e]) @ tp["Wk"][e].T) ** 2
        oe = he @ tp["Wv"][e].T
        we = ((inds == e).to(torch.float64) * g_sel).sum(dim=1, keepdim=True)
        out = out + we * oe
    P = torch.softmax(lg, dim=-1)
    aux = E * torch.sum(f * P.mean(dim=0))
    z = torch.mean(torch.logsumexp(lg, dim=-1) ** 2)
    loss = torch.sum(torch.tensor(dO, dtype=torch.float64).reshape(-1, C) * out) + d_aux * aux + d_z * z
    loss.backward()
    pairs = [("dx", tx.grad), ("dx_prev", txp.grad), ("dx_k", tp["x_k"].grad), ("dWk", tp["Wk"].grad),
             ("dWv", tp["Wv"].grad), ("dWg", tp["Wg"].grad)]
    for name, want in pairs:
        want = want.numpy()
        err = np.max(np.abs(np.asarray(g[name]) - want)) / (np.max(np.abs(want)) + 1e-12)
        assert err < 1e-5, f"{name}: max rel err {err:.3g}"


def test_smooth_forward_matches_forward_oracle():
    Bsz, T, C, F, E, k = 2, 5, 64, 128, 4, 2
    x, p, dO, xp, b = _case(Bsz, T, C, F, E, seed=7, bias=True)
    parts = O.experts_forward(x, p, k, "f32", x_prev=xp, bias=b, return_parts=True)
    _, out, aux, z = MB.experts_smooth_loss(x, p, parts["inds"], parts["counts"], dO, x_prev=xp, bias=b)
    ref = parts["out"].reshape(-1, C).astype(np.float64)
    assert np.max(np.abs(out - ref)) <= 1e-5 * np.max(np.abs(ref))
    assert abs(aux - parts["aux"]) <= 1e-5 * abs(aux)
    assert abs(z - parts["z"]) <= 1e-5 * abs(z)


def test_zero_values_closed_form():
    Bsz, T, C, F, E, k = 1, 6, 64, 64, 3, 2
    x, p, dO, xp, _ = _case(Bsz, T, C, F, E, seed=5)
    p["Wv"][:] = 0
    g = MB.experts_backward(x, p, k, "f32", dO, 0.4, 0.9, x_prev=xp)
    assert np.all(g["dWk"] == 0) and np.all(g["dx_k"] == 0) and np.all(g["dg"] == 0)
    assert np.all(g["dx_prev"] == 0)
    # dx is the router term alone: dℓ·W_gate
    assert np.allclose(g["dx"].reshape(-1, C), g["dlogits"] @ p["Wg"].astype(np.float64), rtol=0, atol=1e-12)
    assert np.any(g["dWv"] != 0)


def test_single_expert_is_the_channel_mix_gradient():
    Bsz, T, C, F, E, k = 1, 5, 64, 128, 1, 1
    x, p, dO, _, _ = _case(Bsz, T, C, F, E, seed=9, prev=False)
    g = MB.experts_backward(x, p, k, "f32", dO, 0.0, 0.0)
    assert np.all(g["dlogits"] == 0) and np.all(g["dWg"] == 0)
    # gate 1: dW_val = hᵀ·dO with h the plain ChannelMix hidden
    h = O.cmix_hidden(x, p["x_k"][0], p["Wk"][0], "f32").reshape(-1, F).astype(np.float64)
    want = dO.reshape(-1, C).astype(np.float64).T @ h
    assert np.allclose(g["dWv"][0], want, rtol=1e-12, atol=1e-12)
