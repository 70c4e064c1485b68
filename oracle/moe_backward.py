"""CPU oracle for the backward (VJP) of the LoRA-MoE ChannelMix layer.

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` as the checker; the product
path never imports it.

The reference trains this layer with MLX autodiff (rwkv_mlx/finetune_moe.py:
215-232, ``nn.value_and_grad`` over moe.py:129-147).  Its VJP with respect
to x, lora_A, lora_B and router.gate.weight, given the cotangents of
(out, aux_loss, z_loss), is restated here in float64 from the forward's
definition:

* the base output is under ``stop_gradient`` (moe.py:131): no gradient
  reaches x, W_key, W_value or x_k through it;
* the top-k selection and the counts f_e (moe.py:66-68, 80-83) are piecewise
  constant: no gradient flows through them;
* casts (``astype``) pass cotangents through unchanged.

With s_e = x·A_e and a_e = s_e·B_e (the forward's rounded values), gates
g = softmax(ℓ[I]) and w_e = Σ_slot [I = e] g (moe.py:69-70, 138-145):

    dg_j      = <dO, a_{e_j}>                       slot j of a token
    da_e      = w_e ⊙ dO
    ds_e      = da_e · B_eᵀ
    dB_e      = s_eᵀ · da_e
    dA_e      = xᵀ · ds_e
    dx       += Σ_e ds_e · A_eᵀ
    dℓ[I_j]  += g_j (dg_j − Σ_i g_i dg_i)            softmax over the selected logits
    dℓ       += d_aux · (E/N) · P ⊙ (f − <P, f>)     aux = E Σ_e f_e mean_t P_e   (moe.py:76-84)
    dℓ       += d_z · (2 lse / N) · P               z = mean_t lse²              (moe.py:61-62)
    dW_gate   = dℓᵀ · x ;  dx += dℓ · W_gate         ℓ = x·W_gateᵀ               (moe.py:56)

with P = softmax(ℓ) and lse = log Σ_e exp ℓ.  ``ortho_grad`` is the gradient
of orthogonal_loss (moe.py:149-163), which the reference's Block adds to the
training loss (model.py:323).  ``layer_norm_backward`` is the VJP of the
Block's ln2 in front of the layer (model.py:321), which a training step
differentiates through.  ``smooth_loss`` is the
forward restated in float64 without the dtype roundings, for finite
differences: tests/test_backward_oracle.py checks every gradient here
against central differences of it, and checks ``smooth_loss``'s pieces
against ``moe_oracle.moe_forward``.
"""
from __future__ import annotations

import numpy as np

from . import moe_oracle as O


def _softmax(v, axis=-1):
    m = v.max(axis=axis, keepdims=True)
    e = np.exp(v - m)
    return e / e.sum(axis=axis, keepdims=True)


def moe_backward(x, Wg, A, B, k, dtype, dO, d_aux=0.0, d_z=0.0, bias=None, gate_dtype=None, adapter_dtype=None):
    """Gradients of <dO, out> + d_aux·aux + d_z·z with respect to x (N,C),
    W_gate (E,C), lora_A (E,C,r) and lora_B (E,r,C), in float64.

    x, Wg, A, B hold dtype values (float32 arrays, as the forward oracle
    takes them); dO (N,C) is the cotangent of out.  The selection, gates and
    s_e, a_e are the forward oracle's: gates rounded to dtype (x's, moe.py:86),
    s_e and a_e rounded to promote(dtype, adapter_dtype) (moe.py:138-147), the
    logits from W_gate of gate_dtype (the fine-tune layer: an fp16 x with an
    fp32 gate and fp32 adapters)."""
    x = np.asarray(x, np.float32)
    N, C = x.shape
    E, _, r = A.shape
    rt = O.router(x, Wg, k, dtype, bias, gate_dtype=gate_dtype)
    ad = O.promote(dtype, adapter_dtype)
    lg = rt["logits"].astype(np.float64)
    inds = rt["inds"]
    gates = rt["gates"].astype(np.float64)        # w_e values of the forward (rounded)
    sel = np.take_along_axis(lg, inds, axis=-1)
    gt = _softmax(sel)                             # the softmax the gates come from
    x64 = x.astype(np.float64)
    dO = np.asarray(dO, np.float64)
    dx = np.zeros((N, C))
    dA = np.zeros((E, C, r))
    dB = np.zeros((E, r, C))
    dg = np.zeros((N, k))
    for e in range(E):
        s_e = O._mm(x, A[e], ad).astype(np.float64)                    # (N, r), rounded like the forward
        a_e = O._mm(s_e.astype(np.float32), B[e], ad).astype(np.float64)     # (N, C)
        w_e = np.where(inds == e, gates, 0.0).sum(axis=-1)             # (N,)
        hit = inds == e
        dg[hit] = np.broadcast_to((dO * a_e).sum(axis=-1)[:, None], hit.shape)[hit]
        da = w_e[:, None] * dO
        ds = da @ B[e].astype(np.float64).T
        dB[e] = s_e.T @ da
        dA[e] = x64.T @ ds
        dx += ds @ A[e].astype(np.float64).T
    dl = _logit_grad(lg, inds, rt["counts"], dg, d_aux, d_z)
    Wg64 = np.asarray(Wg, np.float64)
    dWg = dl.T @ x64
    dx += dl @ Wg64
    return {"dx": dx, "dA": dA, "dB": dB, "dWg": dWg, "dlogits": dl, "dg": dg, "inds": inds}


def _logit_grad(lg, inds, counts, dg, d_aux, d_z):
    """d loss / d logits (N, E) in float64 (moe.py:56-86): the selected-logit
    softmax's Jacobian applied to the slot cotangents dg (N, k), plus the aux
    term d_aux·(E/N)·P⊙(f − <P,f>) and the z term d_z·(2 lse/N)·P, with
    P = softmax(ℓ), lse = log Σ_e exp ℓ and f = counts / (N·k)."""
    N, E = lg.shape
    k = inds.shape[1]
    gt = _softmax(np.take_along_axis(lg, inds, axis=-1))
    dsel = gt * (dg - (gt * dg).sum(axis=-1, keepdims=True))
    dl = np.zeros((N, E))
    np.add.at(dl, (np.arange(N)[:, None].repeat(k, 1), inds), dsel)
    P = _softmax(lg)
    f = np.asarray(counts, np.float64) / (N * k)
    dl += d_aux * (E / N) * P * (f[None, :] - (P * f[None, :]).sum(axis=-1, keepdims=True))
    lse = np.log(np.exp(lg).sum(axis=-1))
    dl += d_z * (2.0 * lse / N)[:, None] * P
    return dl


def router_backward(x, Wg, k, dtype, d_gates, d_aux=0.0, d_z=0.0, bias=None):
    """VJP of the standalone Router (moe.py:35-86): gradients of
    <d_gates, gates> + d_aux·aux + d_z·z with respect to x (N,C) and W_gate
    (E,C), in float64.  The selection and counts are the forward oracle's
    (piecewise constant); the gates' cast to dtype passes the cotangent
    through (so d_gates acts on the unrounded softmax)."""
    x64 = np.asarray(x, np.float64)
    rt = O.router(np.asarray(x, np.float32), Wg, k, dtype, bias)
    lg = rt["logits"].astype(np.float64)
    dl = _logit_grad(lg, rt["inds"], rt["counts"], np.asarray(d_gates, np.float64), d_aux, d_z)
    return {"dx": dl @ np.asarray(Wg, np.float64), "dWg": dl.T @ x64, "dlogits": dl, "inds": rt["inds"]}


def router_smooth_loss(x, Wg, inds, counts, d_gates, d_aux=0.0, d_z=0.0, bias=None):
    """<d_gates, softmax(ℓ[inds])> + d_aux·aux + d_z·z in float64 without
    roundings, for a fixed selection and fixed counts (their values at the
    point of differentiation): the function router_backward differentiates."""
    x = np.asarray(x, np.float64)
    N = x.shape[0]
    E = np.asarray(Wg).shape[0]
    k = inds.shape[1]
    lg = x @ np.asarray(Wg, np.float64).T
    if bias is not None:
        lg = lg + np.asarray(bias, np.float64)[None, :]
    g = _softmax(np.take_along_axis(lg, inds, axis=-1))
    P = _softmax(lg)
    f = np.asarray(counts, np.float64) / (N * k)
    aux = E * float((f * P.mean(axis=0)).sum())
    lse = np.log(np.exp(lg).sum(axis=-1))
    z = float((lse ** 2).mean())
    return float((np.asarray(d_gates, np.float64) * g).sum()) + d_aux * aux + d_z * z


def layer_norm_backward(x, w, dy, eps=1e-5, d_res=None):
    """VJP of the Block's ln2 (model.py:321 with nn.LayerNorm(C), model.py:283):
    y = x̂·w + b with x̂ = (x − mean)·rstd, rstd = 1/sqrt(var + eps), per row
    of x (N, C).  Given dy = d loss / d y, in float64:

        dx = rstd · (g − mean(g) − x̂ · mean(g ⊙ x̂)),   g = dy ⊙ w
        dw = Σ_rows dy ⊙ x̂,   db = Σ_rows dy

    plus d_res (the cotangent of the Block's residual branch x + ffn(ln2(x)),
    model.py:321) added to dx when given.  Pinned against torch autograd of
    layer_norm in float64, central differences and the invariants
    Σ_c dx = 0, Σ_c dx·x̂ = 0 (tests/test_layer_norm_oracle.py)."""
    x = np.asarray(x, np.float64)
    dy = np.asarray(dy, np.float64)
    w = np.asarray(w, np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    rstd = 1.0 / np.sqrt(var + eps)
    xh = (x - mean) * rstd
    g = dy * w[None, :]
    dx = rstd * (g - g.mean(axis=-1, keepdims=True) - xh * (g * xh).mean(axis=-1, keepdims=True))
    if d_res is not None:
        dx = dx + np.asarray(d_res, np.float64)
    return {"dx": dx, "dw": (dy * xh).sum(axis=0), "db": dy.sum(axis=0)}


def ortho_grad(A):
    """d/dA of orthogonal_loss = Σ_{i<j} ||A_iᵀ A_j||_F² (moe.py:149-163), in
    float64: dA_i = 2 Σ_{j≠i} A_j (A_jᵀ A_i)."""
    A = np.asarray(A, np.float64)
    E = A.shape[0]
    out = np.zeros_like(A)
    for i in range(E):
        for j in range(E):
            if j != i:
                out[i] += 2.0 * A[j] @ (A[j].T @ A[i])
    return out


def ortho_loss64(A):
    """orthogonal_loss in float64 without roundings (for finite differences)."""
    A = np.asarray(A, np.float64)
    E = A.shape[0]
    return float(sum(np.sum((A[i].T @ A[j]) ** 2) for i in range(E) for j in range(i + 1, E)))


def smooth_loss(x, Wg, A, B, inds, counts, dO, d_aux=0.0, d_z=0.0, bias=None):
    """<dO, delta> + d_aux·aux + d_z·z in float64 with no roundings, for a
    fixed selection `inds` and fixed counts (their values at the point of
    differentiation).  The base output is a constant under stop_gradient and
    drops out of every derivative."""
    x = np.asarray(x, np.float64)
    N, C = x.shape
    E, _, r = A.shape
    k = inds.shape[1]
    lg = x @ np.asarray(Wg, np.float64).T
    if bias is not None:
        lg = lg + np.asarray(bias, np.float64)[None, :]
    g = _softmax(np.take_along_axis(lg, inds, axis=-1))
    delta = np.zeros((N, C))
    for j in range(k):
        for e in range(E):
            m = inds[:, j] == e
            if m.any():
                delta[m] += g[m, j][:, None] * ((x[m] @ A[e]) @ B[e])
    P = _softmax(lg)
    f = np.asarray(counts, np.float64) / (N * k)
    aux = E * float(np.sum(f * P.mean(axis=0)))
    lse = np.log(np.exp(lg).sum(axis=-1))
    z = float(np.mean(lse * lse))
    return float(np.sum(np.asarray(dO, np.float64) * delta)) + d_aux * aux + d_z * z, delta, aux, z


# ---------------------------------------------------------------------------
# full-expert layer (MoE_CMix, moe.py:170-242)
# ---------------------------------------------------------------------------

def experts_backward(x, p, k, dtype, dO, d_aux=0.0, d_z=0.0, x_prev=None, bias=None):
    """Gradients of <dO, out> + d_aux·aux + d_z·z for MoE_CMix.__call__
    (moe.py:218-234) with respect to x (B,T,C), the carried shift state
    x_prev (B,C) when given, x_k (E,C), expert_key (E,F,C), expert_val
    (E,C,F) and router.gate.weight (E,C), in float64.  Every parameter is
    trainable (the full-expert layer has no stop_gradient).

    For expert e, with the forward's rounded values xx = shift(x) − x,
    k_e = x + xx·μ_e, p_e = k_e·W_key,eᵀ, h_e = relu(p_e)², o_e = h_e·W_val,eᵀ
    and the dense gate w_e = Σ_slot [I = e]·g (moe.py:226-233):

        dg_j      = <dO, o_{e_j}>                       slot j of a token
        do_e      = w_e ⊙ dO
        dW_val,e  = do_eᵀ · h_e
        dp_e      = (do_e · W_val,e) ⊙ 2·relu(p_e)
        dW_key,e  = dp_eᵀ · k_e
        dk_e      = dp_e · W_key,e
        dx       += dk_e ⊙ (1 − μ_e) ;  d shift(x) += dk_e ⊙ μ_e ;  dμ_e = Σ_t dk_e ⊙ xx

    (a token's shift input is x[t−1] inside its sequence and x_prev at its
    start), and the router terms as in ``moe_backward``."""
    x = np.asarray(x, np.float32)
    Bsz, T, C = x.shape
    N = Bsz * T
    E = p["Wg"].shape[0]
    flat = x.reshape(N, C)
    rt = O.router(flat, p["Wg"], k, dtype, bias)
    lg = rt["logits"].astype(np.float64)
    inds = rt["inds"]
    gates = rt["gates"].astype(np.float64)
    gt = _softmax(np.take_along_axis(lg, inds, axis=-1))
    dO = np.asarray(dO, np.float64).reshape(N, C)
    prev = O.time_shift(x, None if x_prev is None else np.asarray(x_prev, np.float32))
    xx = O.round_to(prev - x, dtype).reshape(N, C)
    xx64 = xx.astype(np.float64)
    dx = np.zeros((N, C))
    dshift = np.zeros((N, C))
    dmu = np.zeros((E, C))
    dWk = np.zeros(p["Wk"].shape)
    dWv = np.zeros(p["Wv"].shape)
    dg = np.zeros((N, k))
    for e in range(E):
        mu = np.asarray(p["x_k"][e], np.float32).reshape(-1)
        k_e = O.round_to(flat + O.round_to(xx * mu, dtype), dtype)
        p_e = O._mm(k_e, np.asarray(p["Wk"][e], np.float32).T, dtype).astype(np.float64)
        rp = np.maximum(p_e, 0.0)
        h_e = O.round_to(rp * rp, dtype).astype(np.float64)
        o_e = O._mm(h_e.astype(np.float32), np.asarray(p["Wv"][e], np.float32).T, dtype).astype(np.float64)
        w_e = np.where(inds == e, gates, 0.0).sum(axis=-1)
        hit = inds == e
        dg[hit] = np.broadcast_to((dO * o_e).sum(axis=-1)[:, None], hit.shape)[hit]
        do = w_e[:, None] * dO
        dWv[e] = do.T @ h_e
        dp = (do @ np.asarray(p["Wv"][e], np.float64)) * 2.0 * rp
        dWk[e] = dp.T @ k_e.astype(np.float64)
        dk = dp @ np.asarray(p["Wk"][e], np.float64)
        mu64 = mu.astype(np.float64)
        dx += dk * (1.0 - mu64)[None, :]
        dshift += dk * mu64[None, :]
        dmu[e] = (dk * xx64).sum(axis=0)
    # shift(x)[t] is x[t-1] inside a sequence, x_prev (or 0) at its start
    ds = dshift.reshape(Bsz, T, C)
    dx3 = dx.reshape(Bsz, T, C)
    dx3[:, :-1] += ds[:, 1:]
    dx_prev = ds[:, 0].copy() if x_prev is not None else None
    dx = dx3.reshape(N, C)
    dsel = gt * (dg - (gt * dg).sum(axis=-1, keepdims=True))
    dl = np.zeros((N, E))
    np.add.at(dl, (np.arange(N)[:, None].repeat(k, 1), inds), dsel)
    P = _softmax(lg)
    f = rt["counts"].astype(np.float64) / (N * k)
    dl += d_aux * (E / N) * P * (f[None, :] - (P * f[None, :]).sum(axis=-1, keepdims=True))
    lse = np.log(np.exp(lg).sum(axis=-1))
    dl += d_z * (2.0 * lse / N)[:, None] * P
    Wg64 = np.asarray(p["Wg"], np.float64)
    dWg = dl.T @ flat.astype(np.float64)
    dx += dl @ Wg64
    return {"dx": dx.reshape(Bsz, T, C), "dx_prev": dx_prev, "dx_k": dmu, "dWk": dWk, "dWv": dWv, "dWg": dWg,
            "dlogits": dl, "dg": dg, "inds": inds}


def experts_smooth_loss(x, p, inds, counts, dO, d_aux=0.0, d_z=0.0, x_prev=None, bias=None):
    """<dO, out> + d_aux·aux + d_z·z of MoE_CMix in float64 with no roundings,
    for a fixed selection `inds` and counts (for finite differences)."""
    x = np.asarray(x, np.float64)
    Bsz, T, C = x.shape
    N = Bsz * T
    E = np.asarray(p["Wg"]).shape[0]
    k = inds.shape[1]
    flat = x.reshape(N, C)
    lg = flat @ np.asarray(p["Wg"], np.float64).T
    if bias is not None:
        lg = lg + np.asarray(bias, np.float64)[None, :]
    g = _softmax(np.take_along_axis(lg, inds, axis=-1))
    prev = np.zeros_like(x)
    prev[:, 1:] = x[:, :-1]
    if x_prev is not None:
        prev[:, 0] = np.asarray(x_prev, np.float64)
    xx = (prev - x).reshape(N, C)
    out = np.zeros((N, C))
    for j in range(k):
        for e in range(E):
            m = inds[:, j] == e
            if m.any():
                ke = flat[m] + xx[m] * np.asarray(p["x_k"][e], np.float64)[None, :]
                he = np.maximum(ke @ np.asarray(p["Wk"][e], np.float64).T, 0.0) ** 2
                out[m] += g[m, j][:, None] * (he @ np.asarray(p["Wv"][e], np.float64).T)
    P = _softmax(lg)
    f = np.asarray(counts, np.float64) / (N * k)
    aux = E * float(np.sum(f * P.mean(axis=0)))
    lse = np.log(np.exp(lg).sum(axis=-1))
    z = float(np.mean(lse * lse))
    return float(np.sum(np.asarray(dO, np.float64).reshape(N, C) * out)) + d_aux * aux + d_z * z, out, aux, z
