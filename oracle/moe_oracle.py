"""CPU oracle for the LoRA-MoE ChannelMix forward.

TEST INFRASTRUCTURE ONLY.  This module is imported by ``tests/``, by
``__graft_entry__.smoke()`` as the checker, and by ``bench.py``'s
``cpu_baseline`` leg.  The product path (``rwkv_mlx_amd``) never imports it.

It restates, in NumPy, the algorithm of the reference's MLX code:

* ``time_shift``         rwkv_mlx/model.py:67-75
* ``cmix_base``          rwkv_mlx/model.py:243-263 (RWKV_CMix_x070.__call__)
* ``cmix_decode``        rwkv_mlx/model.py:498-506 (_channel_mixing_rnn)
* ``router``             rwkv_mlx/moe.py:51-86     (Router.__call__)
* ``lora_delta_dense``   rwkv_mlx/moe.py:138-145   (the dense masked expert loop)
* ``moe_forward``        rwkv_mlx/moe.py:129-147   (LoRAMoE_CMix.__call__)
* ``ortho_loss``         rwkv_mlx/moe.py:149-163   (orthogonal_loss)
* ``experts_forward``    rwkv_mlx/moe.py:218-234   (MoE_CMix.__call__, the dense expert loop)
* ``layer_norm``         rwkv_mlx/model.py:283, 321 (Block.ln2, nn.LayerNorm) and
                         model.py:434-438 (_layer_norm_1d, the RNN form)
* ``dispatch``           no reference counterpart: the stable counting sort
                         that replaces moe.py's masks (closed form).

Numerics.  Arrays are carried as float32 holding values of the layer dtype
("f32", "f16" or "bf16").  Each reference op on dtype-typed arrays is
rounded to the dtype, as MLX does: products are computed in ``mm_dtype``
(float64 by default, so the oracle sits closer to the exact value than any
fp32 implementation) and rounded once.  Router logits follow an exact,
order-fixed definition (see ``router_logits``) that the GPU reproduces bit for
bit.

Parity pins (tests/test_oracle.py): bf16/fp16 rounding against torch's casts;
logits against a pure-Python loop and exact rational sums; top-k against a
brute-force sort; gates, z and aux against closed forms; dispatch against a
brute-force stable sort; base, LoRA and decode against pure-Python loops on
tiny shapes and against special cases (x_k = 0 / 1, B = 0, identical
experts); ortho against orthogonal / identical column spaces; and all of it
against the float64 known-answer fixtures in tests/golden/.
"""
from __future__ import annotations

import numpy as np

DTYPES = ("f32", "f16", "bf16")


# ---------------------------------------------------------------------------
# rounding
# ---------------------------------------------------------------------------

def bf16_round(a) -> np.ndarray:
    """Round float32 values to bfloat16 (round to nearest, ties to even)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).copy()
    nan = np.isnan(a)
    if nan.any():
        out[nan] = np.float32("nan")
    return out.reshape(a.shape)


def round_to(a, dtype: str) -> np.ndarray:
    """Round to the layer dtype, returned as float32."""
    a = np.asarray(a, dtype=np.float32)
    if dtype == "f32":
        return a
    if dtype == "f16":
        return a.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return bf16_round(a)
    raise ValueError(f"unknown dtype {dtype!r}")


def promote(*dtypes: str | None) -> str:
    """MLX type promotion among the layer dtypes (None entries are skipped):
    float32 wins; float16 with bfloat16 gives float32; otherwise the common
    dtype."""
    ds = {d for d in dtypes if d is not None}
    if not ds:
        raise ValueError("no dtype")
    if len(ds) == 1:
        return ds.pop()
    return "f32"


def _mm(a, b, dtype: str, mm_dtype=np.float64) -> np.ndarray:
    """MLX matmul on dtype arrays: exact-ish product, one rounding to dtype."""
    return round_to(np.matmul(np.asarray(a, mm_dtype), np.asarray(b, mm_dtype)), dtype)


# ---------------------------------------------------------------------------
# base ChannelMix (model.py:67-75, 243-263, 498-506)
# ---------------------------------------------------------------------------

def layer_norm(x, w, b, dtype: str, eps: float = 1e-5) -> np.ndarray:
    """ln2 in front of the ChannelMix (model.py:321 with nn.LayerNorm(C),
    model.py:283; the RNN form _layer_norm_1d, model.py:434-438): per row,
    mean and rstd = 1 / sqrt(var + eps), var = mean((x - mean)^2), in
    float64, rounded to float32; then y = ((x - mean) * rstd) * w + b in
    float32, one rounding per operation, rounded to dtype.  MLX evaluates
    nn.LayerNorm in fp32 (mx.fast.layer_norm) and _layer_norm_1d op by op in
    the row's dtype; both sit within the dtype tolerance of this value.
    Pinned against torch.nn.functional.layer_norm in float64 and closed forms
    (tests/test_layer_norm_oracle.py)."""
    x64 = np.asarray(x, dtype=np.float64)
    mean = x64.sum(axis=-1, keepdims=True) / x64.shape[-1]
    d64 = x64 - mean
    var = (d64 * d64).sum(axis=-1, keepdims=True) / x64.shape[-1]
    rstd = 1.0 / np.sqrt(var + eps)
    x32 = np.asarray(x, dtype=np.float32)
    d = (x32 - mean.astype(np.float32)) * rstd.astype(np.float32)
    y = d * np.asarray(w, dtype=np.float32) + np.asarray(b, dtype=np.float32)
    return round_to(y, dtype)


def time_shift(x: np.ndarray, x_prev: np.ndarray | None = None) -> np.ndarray:
    """shift(x)[:, t] = x[:, t-1]; row 0 is zeros (model.py:73-75) or the
    carried state x_prev (RNN mode)."""
    prev = np.zeros_like(x)
    prev[:, 1:] = x[:, :-1]
    if x_prev is not None:
        prev[:, 0] = x_prev
    return prev


def cmix_hidden(x, x_k, Wk, dtype, x_prev=None, mm_dtype=np.float64):
    """k = relu(key(x + (shift(x) - x) * x_k)) ** 2 (model.py:260-262)."""
    x = np.asarray(x, np.float32)
    mu = np.asarray(x_k, np.float32).reshape(-1)
    xx = round_to(time_shift(x, x_prev) - x, dtype)
    xk = round_to(x + round_to(xx * mu, dtype), dtype)
    h = _mm(xk, np.asarray(Wk, np.float32).T, dtype, mm_dtype)
    h = np.maximum(h, 0.0)
    return round_to(h * h, dtype)


def cmix_base(x, x_k, Wk, Wv, dtype, x_prev=None, mm_dtype=np.float64):
    """RWKV_CMix_x070.__call__ (model.py:259-263): value(relu(key(xk))**2)."""
    h = cmix_hidden(x, x_k, Wk, dtype, x_prev, mm_dtype)
    return _mm(h, np.asarray(Wv, np.float32).T, dtype, mm_dtype)


def cmix_decode(x, x_prev, x_k, Wk, Wv, dtype, mm_dtype=np.float64):
    """_channel_mixing_rnn (model.py:498-506) on a batch of single tokens:
    returns (out, new_state = x)."""
    x = np.asarray(x, np.float32)
    xx = round_to(np.asarray(x_prev, np.float32) - x, dtype)
    k = round_to(x + round_to(xx * np.asarray(x_k, np.float32).reshape(-1), dtype), dtype)
    h = np.maximum(_mm(k, np.asarray(Wk, np.float32).T, dtype, mm_dtype), 0.0)
    h = round_to(h * h, dtype)
    return _mm(h, np.asarray(Wv, np.float32).T, dtype, mm_dtype), x


# ---------------------------------------------------------------------------
# router (moe.py:51-86)
# ---------------------------------------------------------------------------

def logit_acc(dtype: str) -> str:
    """Accumulator of the router's chunk sums for a layer dtype: fp32 for
    fp16/bf16 inputs (their products are exact in fp32), fp64 for fp32 inputs."""
    return "f64" if dtype == "f32" else "f32"


def router_logits(x, Wg, bias=None, acc="f64") -> np.ndarray:
    """logits[t, e] = fp32(Σ_q Σ_{j<64} x[t, 64q+j]·Wg[e, 64q+j]) (+ bias[e]).

    The inner sums run in ascending j from 0, one fused multiply-add per term
    in the accumulator format `acc` ("f64", or "f32" for fp16/bf16 inputs).
    The chunk partials are summed in float64 in ascending q from 0.0, and the
    total is rounded once to float32.  The product of two inputs is exact in
    the accumulator format, so each step is one IEEE rounding and the result
    is a function of the inputs alone.  An fp32 FMA is computed here as the
    float64 sum of the exact product and the fp32 accumulator rounded to fp32,
    which equals the fused result (float64 has more than 2·24 + 2 bits).
    moe.py:56 computes the same dot product in fp32, in an order MLX does not
    specify.
    """
    x = np.asarray(x, np.float32)
    lead = x.shape[:-1]
    C = x.shape[-1]
    if C % 64:
        raise ValueError("d_model must be a multiple of 64")
    if acc not in ("f64", "f32"):
        raise ValueError(f"unknown accumulator {acc!r}")
    Wg = np.asarray(Wg, np.float32)
    E = Wg.shape[0]
    Q = C // 64
    x64 = x.reshape(-1, Q, 64).astype(np.float64)
    w64 = Wg.reshape(E, Q, 64).astype(np.float64)
    acc_dt = np.float64 if acc == "f64" else np.float32
    acc = np.zeros((x64.shape[0], E, Q), acc_dt)
    for j in range(64):
        acc = (acc.astype(np.float64) + x64[:, None, :, j] * w64[None, :, :, j]).astype(acc_dt)
    acc = acc.astype(np.float64)
    tot = np.zeros((x64.shape[0], E), np.float64)
    for q in range(Q):
        tot += acc[:, :, q]
    logits = tot.astype(np.float32)
    if bias is not None:
        logits = (logits + np.asarray(bias, np.float32)[None, :]).astype(np.float32)
    return logits.reshape(*lead, E)


def topk_canonical(logits: np.ndarray, k: int) -> np.ndarray:
    """The k largest logits per row, in descending order, ties to the lower id.

    For k <= 2 this is exactly argpartition(-logits, kth=k-1)[..., :k]
    (moe.py:66-68); for k >= 3 MLX leaves the first k-1 slots unordered and
    this fixes them to descending order."""
    return np.argsort(-logits, axis=-1, kind="stable")[..., :k].astype(np.int32)


def router(x, Wg, k, dtype, bias=None, gate_dtype=None):
    """Router.__call__ (moe.py:51-86).

    ``dtype`` is x's dtype; ``gate_dtype`` that of gate.weight (default: the
    same).  The logits are fp32(x)·fp32(W) (moe.py:56): with an fp32 operand
    the chunk sums use the fp64 definition (the product of an fp32 value and
    a 16-bit or fp32 value is exact in fp64).  Gates are cast to x's dtype
    (moe.py:86).

    Returns dict with logits (N,E) fp32, inds (N,k) int32, gates (N,k) in
    dtype, aux and z (python floats) and the per-expert counts."""
    logits = router_logits(x, Wg, bias, acc=logit_acc(promote(dtype, gate_dtype)))
    E = logits.shape[-1]
    lg = logits.reshape(-1, E)
    N = lg.shape[0]
    # z-loss: mean over tokens of (log Σ_e exp ℓ)², no max shift (moe.py:61-62);
    # logits above ~88.7 overflow to inf there too
    with np.errstate(over="ignore"):
        lse = np.log(np.exp(lg).sum(axis=-1, dtype=np.float32)).astype(np.float32)
    z = float(np.mean((lse * lse).astype(np.float64)))
    inds = topk_canonical(lg, k)
    sel = np.take_along_axis(lg, inds, axis=-1)
    ex = np.exp(sel - sel[:, :1]).astype(np.float32)
    gates = round_to(ex / ex.sum(axis=-1, keepdims=True, dtype=np.float32), dtype)
    # load balance (moe.py:76-84)
    m = lg.max(axis=-1, keepdims=True)
    pe = np.exp(lg - m).astype(np.float32)
    probs = pe / pe.sum(axis=-1, keepdims=True, dtype=np.float32)
    p_e = probs.astype(np.float64).mean(axis=0)
    counts = np.bincount(inds.reshape(-1), minlength=E)
    f_e = counts.astype(np.float64) / (N * k)
    aux = float(E * np.sum(f_e * p_e))
    return {"logits": lg, "inds": inds, "gates": gates, "aux": aux, "z": z, "counts": counts}


def gate_dense(inds, gates, E):
    """w_e = Σ_slot [inds == e]·g (moe.py:144) for every expert: (N, E)."""
    N, k = inds.shape
    g = np.zeros((N, E), np.float32)
    for s in range(k):
        g[np.arange(N), inds[:, s]] += gates[:, s]
    return g


# ---------------------------------------------------------------------------
# dispatch (stable counting sort; no reference counterpart)
# ---------------------------------------------------------------------------

def dispatch(inds: np.ndarray, E: int):
    """perm: assignment ids a = t*k + slot sorted stably by expert id;
    inv_perm[a] = position of a; offsets = exclusive cumsum of counts."""
    flat = np.asarray(inds, np.int64).reshape(-1)
    perm = np.argsort(flat, kind="stable").astype(np.int32)
    inv = np.empty_like(perm)
    inv[perm] = np.arange(perm.size, dtype=np.int32)
    counts = np.bincount(flat, minlength=E)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    return perm, inv, offsets


# ---------------------------------------------------------------------------
# LoRA experts and the full module (moe.py:129-163)
# ---------------------------------------------------------------------------

def lora_adapter(x, A_e, B_e, dtype, mm_dtype=np.float64):
    """(x @ A_e) @ B_e with both products rounded to dtype (moe.py:142)."""
    return _mm(_mm(x, A_e, dtype, mm_dtype), B_e, dtype, mm_dtype)


def lora_delta_dense(x, A, B, inds, gates, dtype, mm_dtype=np.float64):
    """The literal expert loop of moe.py:138-145 on (N, C) rows; ``dtype`` is
    the adapters' compute dtype (promote(x, lora_A, lora_B))."""
    N, C = x.shape
    E = A.shape[0]
    delta = np.zeros((N, C), np.float32)
    for e in range(E):
        adapter = lora_adapter(x, A[e], B[e], dtype, mm_dtype)
        w_e = np.where(inds == e, gates, 0.0).sum(axis=-1, keepdims=True).astype(np.float32)
        delta = round_to(delta + round_to(w_e * adapter, dtype), dtype)
    return delta


def lora_delta_sparse(x, A, B, inds, gates, dtype, mm_dtype=np.float64):
    """Same value as lora_delta_dense, evaluated only on routed rows through
    the dispatch permutation (the GPU SPARSE mode's algorithm)."""
    N, C = x.shape
    E = A.shape[0]
    k = inds.shape[1]
    perm, _, offsets = dispatch(inds, E)
    rows = np.zeros((N * k, C), np.float32)
    for e in range(E):
        sl = perm[offsets[e]:offsets[e + 1]]
        if sl.size:
            rows[offsets[e]:offsets[e + 1]] = lora_adapter(x[sl // k], A[e], B[e], dtype, mm_dtype)
    delta = np.zeros((N, C), np.float32)
    pos = np.empty(N * k, np.int64)
    pos[perm] = np.arange(N * k)
    order = np.argsort(inds, axis=1, kind="stable")  # ascending expert per token
    for j in range(k):
        s = order[:, j]
        a = np.arange(N) * k + s
        g = gates[np.arange(N), s][:, None]
        delta = round_to(delta + round_to(g * rows[pos[a]], dtype), dtype)
    return delta


def moe_forward(x, p, k, dtype, x_prev=None, bias=None, mm_dtype=np.float64, return_parts=False,
                gate_dtype=None, adapter_dtype=None):
    """LoRAMoE_CMix.__call__ (moe.py:129-147) on x (B, T, C).

    ``p`` holds x_k (C,), Wk (F,C), Wv (C,F), Wg (E,C), A (E,C,r), B (E,r,C).
    ``dtype`` is the dtype of x and the base; ``gate_dtype`` and
    ``adapter_dtype`` (default: the same) those of router.gate.weight and of
    lora_A / lora_B.  MLX promotion then fixes every rounding point: the base
    runs in dtype (model.py:259-263), the gates are cast to dtype
    (moe.py:86), and (x @ A_e) @ B_e, w_e·adapter, the delta and
    out = base + delta run in promote(dtype, adapter_dtype) (moe.py:138-147),
    e.g. fp32 for the reference's fine-tune layer (fp16 base from convert.py,
    fp32 adapters and gate from moe.py:47, 124-125).
    Returns (out, aux, z) or, with return_parts, a dict with every stage."""
    x = np.asarray(x, np.float32)
    Bsz, T, C = x.shape
    ad = promote(dtype, adapter_dtype)
    base = cmix_base(x, p["x_k"], p["Wk"], p["Wv"], dtype, x_prev, mm_dtype)
    r = router(x.reshape(-1, C), p["Wg"], k, dtype, bias, gate_dtype)
    delta = lora_delta_dense(x.reshape(-1, C), p["A"], p["B"], r["inds"], r["gates"], ad, mm_dtype)
    out = round_to(base.reshape(-1, C) + delta, ad).reshape(Bsz, T, C)
    if return_parts:
        return {"out": out, "base": base.reshape(-1, C), "delta": delta, **r}
    return out, r["aux"], r["z"]


def experts_forward(x, p, k, dtype, x_prev=None, bias=None, mm_dtype=np.float64, return_parts=False):
    """MoE_CMix.__call__ (moe.py:218-234): the router, then the reference's
    dense loop — for e = 0..E-1 the expert ChannelMix on every token
    (token shift with x_k[e], key, relu², value), masked by its dense gate
    w_e = Σ_slot [inds == e]·g, added in ascending e with each product and
    sum rounded to dtype.

    ``p`` holds x_k (E,C), Wk (E,F,C), Wv (E,C,F), Wg (E,C)."""
    x = np.asarray(x, np.float32)
    Bsz, T, C = x.shape
    E = p["Wg"].shape[0]
    r = router(x.reshape(-1, C), p["Wg"], k, dtype, bias)
    out = np.zeros((Bsz * T, C), np.float32)
    for e in range(E):
        base_e = cmix_base(x, p["x_k"][e], p["Wk"][e], p["Wv"][e], dtype, x_prev, mm_dtype).reshape(-1, C)
        w_e = np.where(r["inds"] == e, r["gates"], 0.0).sum(axis=-1, keepdims=True).astype(np.float32)
        out = round_to(out + round_to(w_e * base_e, dtype), dtype)
    out = out.reshape(Bsz, T, C)
    if return_parts:
        return {"out": out, **r}
    return out, r["aux"], r["z"]


def experts_rows(x, p, k, dtype, rows, router_out, x_prev=None, mm_dtype=np.float64):
    """experts_forward's output for the given flat token rows, evaluating only
    each row's routed experts (a row's true predecessor is its shift state)."""
    x = np.asarray(x, np.float32)
    Bsz, T, C = x.shape
    flat = x.reshape(-1, C)
    prev = np.zeros((rows.size, C), np.float32)
    for i, rr in enumerate(rows):
        t = rr % T
        if t > 0:
            prev[i] = flat[rr - 1]
        elif x_prev is not None:
            prev[i] = x_prev[rr // T]
    inds, gates = router_out["inds"][rows], router_out["gates"][rows]
    out = np.zeros((rows.size, C), np.float32)
    order = np.argsort(inds, axis=1, kind="stable")  # ascending expert per row
    for j in range(k):
        s = order[:, j]
        e_r = inds[np.arange(rows.size), s]
        g = gates[np.arange(rows.size), s][:, None]
        contrib = np.zeros((rows.size, C), np.float32)
        for e in np.unique(e_r):
            m = e_r == e
            contrib[m] = cmix_base(flat[rows[m]][:, None, :], p["x_k"][e], p["Wk"][e], p["Wv"][e], dtype,
                                   x_prev=prev[m], mm_dtype=mm_dtype).reshape(-1, C)
        out = round_to(out + round_to(g * contrib, dtype), dtype)
    return out


def ortho_loss(A, dtype, mm_dtype=np.float64) -> float:
    """Σ_{i<j} ||A_iᵀ A_j||_F² (moe.py:149-163); cross and squares rounded to dtype."""
    A = np.asarray(A, np.float32)
    E = A.shape[0]
    total = 0.0
    for i in range(E):
        for j in range(i + 1, E):
            cross = _mm(A[i].T, A[j], dtype, mm_dtype)
            total += float(np.sum(round_to(cross * cross, dtype), dtype=np.float64))
    return total
