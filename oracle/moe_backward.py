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
training loss (model.py:323).  ``smooth_loss`` is the
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


def moe_backward(x, Wg, A, B, k, dtype, dO, d_aux=0.0, d_z=0.0, bias=None):
    """Gradients of <dO, out> + d_aux·aux + d_z·z with respect to x (N,C),
    W_gate (E,C), lora_A (E,C,r) and lora_B (E,r,C), in float64.

    x, Wg, A, B hold dtype values (float32 arrays, as the forward oracle
    takes them); dO (N,C) is the cotangent of out.  The selection, gates and
    s_e, a_e are the forward oracle's (rounded to dtype)."""
    x = np.asarray(x, np.float32)
    N, C = x.shape
    E, _, r = A.shape
    rt = O.router(x, Wg, k, dtype, bias)
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
        s_e = O._mm(x, A[e], dtype).astype(np.float64)                 # (N, r), rounded like the forward
        a_e = O._mm(s_e.astype(np.float32), B[e], dtype).astype(np.float64)  # (N, C)
        w_e = np.where(inds == e, gates, 0.0).sum(axis=-1)             # (N,)
        hit = inds == e
        dg[hit] = np.broadcast_to((dO * a_e).sum(axis=-1)[:, None], hit.shape)[hit]
        da = w_e[:, None] * dO
        ds = da @ B[e].astype(np.float64).T
        dB[e] = s_e.T @ da
        dA[e] = x64.T @ ds
        dx += ds @ A[e].astype(np.float64).T
    dsel = gt * (dg - (gt * dg).sum(axis=-1, keepdims=True))
    dl = np.zeros((N, E))
    np.add.at(dl, (np.arange(N)[:, None].repeat(k, 1), inds), dsel)
    P = _softmax(lg)
    f = rt["counts"].astype(np.float64) / (N * k)
    dl += d_aux * (E / N) * P * (f[None, :] - (P * f[None, :]).sum(axis=-1, keepdims=True))
    lse = np.log(np.exp(lg).sum(axis=-1))
    dl += d_z * (2.0 * lse / N)[:, None] * P
    Wg64 = np.asarray(Wg, np.float64)
    dWg = dl.T @ x64
    dx += dl @ Wg64
    return {"dx": dx, "dA": dA, "dB": dB, "dWg": dWg, "dlogits": dl, "dg": dg, "inds": inds}


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
