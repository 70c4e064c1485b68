#!/usr/bin/env python3
"""Known-answer fixtures for the LoRA-MoE ChannelMix forward, computed by a
brute-force implementation that shares no code with the oracle.

The reference ships no golden vectors and cannot be imported here (it needs
MLX).  These fixtures restate rwkv_mlx/moe.py:51-163 and
rwkv_mlx/model.py:67-75, 259-263, 498-506 with pure-Python loops: every dot
product is an exact rational (fractions.Fraction) rounded once to the layer
dtype, elementwise ops are rounded after each op as MLX does on typed arrays,
and the router logits follow their order-fixed chunked definition (64-wide
chunks, ascending, one fused multiply-add per term in fp32 for fp16/bf16
layers and in fp64 for fp32 layers, chunks summed in fp64).  Every fp32 FMA
here is an exact rational rounded once to fp32 by r32_exact, with no float
arithmetic in between.  Shapes are tiny so the loops finish in seconds.

Run:  python tests/golden/make_fixtures.py   (writes tests/golden/*.npz)
"""
from __future__ import annotations

import math
import struct
from fractions import Fraction
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent


# ---- scalar rounding, independent of numpy's casts --------------------------

def r32(v: float) -> float:
    return struct.unpack("<f", struct.pack("<f", v))[0]


def r16(v: float) -> float:
    return struct.unpack("<e", struct.pack("<e", v))[0]


def rbf16(v: float) -> float:
    """float -> bfloat16 (round to nearest even), via the fp32 bit pattern
    after an exact-to-fp32 rounding of the fp64 value."""
    f = r32(v)
    u = struct.unpack("<I", struct.pack("<f", f))[0]
    lsb = (u >> 16) & 1
    u = (u + 0x7FFF + lsb) & 0xFFFF0000
    return struct.unpack("<f", struct.pack("<I", u))[0]


def rnd(v, dtype: str) -> float:
    v = float(v)
    if dtype == "f32":
        return r32(v)
    if dtype == "f16":
        return r16(v)
    return rbf16(v)


def rnd_exact(q: Fraction, dtype: str) -> float:
    """Round an exact rational to the dtype (via the nearest float64 first;
    a double rounding only where fp64 lands exactly on a dtype tie)."""
    return rnd(float(q), dtype)


def r32_exact(q: Fraction) -> float:
    """An exact rational rounded to the nearest fp32 (ties to even), by
    integer arithmetic; fp32 normal and subnormal range."""
    if q == 0:
        return 0.0
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)                      # below: subnormal spacing
    ulp = Fraction(2) ** (e - 23)
    m = a / ulp
    fl = m.numerator // m.denominator
    rem = m - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return sign * float(fl * ulp)


def dot_exact(a, b) -> Fraction:
    s = Fraction(0)
    for x, y in zip(a, b):
        s += Fraction(x) * Fraction(y)
    return s


# ---- the forward, brute force ----------------------------------------------

def promote(*dts):
    """MLX promotion of float dtypes: fp32 wins, fp16 with bf16 gives fp32."""
    ds = set(dts)
    return ds.pop() if len(ds) == 1 else "f32"


def forward(x, p, k, dtype, x_prev=None, bias=None, gate_dtype=None, adapter_dtype=None):
    """dtype: x and the base weights; gate_dtype / adapter_dtype: router.gate
    and lora_A / lora_B (default: dtype).  Rounding points follow MLX
    promotion: the router dot product is fp32(x)·fp32(W) (moe.py:56), gates
    are cast to x's dtype (moe.py:86), and the adapter products, w_e·adapter,
    the delta and base + delta run in promote(dtype, adapter_dtype)."""
    gate_dtype = gate_dtype or dtype
    ad = promote(dtype, adapter_dtype or dtype)
    B, T, C = len(x), len(x[0]), len(x[0][0])
    xk_mix = p["x_k"]
    Wk, Wv, Wg, A, Bm = p["Wk"], p["Wv"], p["Wg"], p["A"], p["B"]
    F, E, r = len(Wk), len(Wg), len(A[0][0])
    base = [[None] * T for _ in range(B)]
    for b in range(B):
        for t in range(T):
            if t > 0:
                prev = x[b][t - 1]
            elif x_prev is not None:
                prev = x_prev[b]
            else:
                prev = [0.0] * C
            xx = [rnd(prev[c] - x[b][t][c], dtype) for c in range(C)]
            kin = [rnd(x[b][t][c] + rnd(xx[c] * xk_mix[c], dtype), dtype) for c in range(C)]
            h = []
            for f in range(F):
                v = rnd_exact(dot_exact(kin, Wk[f]), dtype)
                v = max(v, 0.0)
                h.append(rnd(v * v, dtype))
            base[b][t] = [rnd_exact(dot_exact(h, Wv[c]), dtype) for c in range(C)]
    # router
    tokens = [x[b][t] for b in range(B) for t in range(T)]
    N = len(tokens)
    logits, inds, gates = [], [], []
    zsum = 0.0
    psum = [0.0] * E
    counts = [0] * E
    for tok in tokens:
        row = []
        for e in range(E):
            tot = 0.0
            for q in range(C // 64):
                acc = 0.0
                for j in range(64):
                    if promote(dtype, gate_dtype) == "f32":  # fp64 FMA: a product with an fp32 factor is exact in fp64
                        acc = acc + tok[64 * q + j] * Wg[e][64 * q + j]
                    else:               # fp32 FMA, rounded once from the exact value
                        acc = r32_exact(Fraction(acc) + Fraction(tok[64 * q + j]) * Fraction(Wg[e][64 * q + j]))
                tot = tot + acc
            v = r32(tot)
            if bias is not None:
                v = r32(v + bias[e])
            row.append(v)
        logits.append(row)
        order = sorted(range(E), key=lambda e: (-row[e], e))
        sel = order[:k]
        inds.append(sel)
        m = row[sel[0]]
        ex = [math.exp(row[e] - m) for e in sel]
        den = sum(ex)
        gates.append([rnd(v / den, dtype) for v in ex])
        lse = math.log(sum(math.exp(v) for v in row))
        zsum += lse * lse
        mx = max(row)
        pe = [math.exp(v - mx) for v in row]
        sp = sum(pe)
        for e in range(E):
            psum[e] += pe[e] / sp
        for e in sel:
            counts[e] += 1
    z = zsum / N
    aux = E * sum((counts[e] / (N * k)) * (psum[e] / N) for e in range(E))
    # experts: the dense masked loop of moe.py:138-145
    out = []
    delta_all = []
    for n, tok in enumerate(tokens):
        delta = [0.0] * C
        for e in range(E):
            u = [rnd_exact(dot_exact(tok, [A[e][c][j] for c in range(C)]), ad) for j in range(r)]
            a_e = [rnd_exact(dot_exact(u, [Bm[e][j][c] for j in range(r)]), ad) for c in range(C)]
            w = sum(g for s, g in zip(inds[n], gates[n]) if s == e)
            delta = [rnd(delta[c] + rnd(w * a_e[c], ad), ad) for c in range(C)]
        b, t = divmod(n, T)
        out.append([rnd(base[b][t][c] + delta[c], ad) for c in range(C)])
        delta_all.append(delta)
    # orthogonality loss (moe.py:149-163)
    ortho = 0.0
    for i in range(E):
        for j in range(i + 1, E):
            for a in range(r):
                for bb in range(r):
                    cr = rnd_exact(dot_exact([A[i][c][a] for c in range(C)], [A[j][c][bb] for c in range(C)]),
                                   adapter_dtype or dtype)
                    ortho += rnd(cr * cr, adapter_dtype or dtype)
    return {"out": out, "base": [v for b in range(B) for v in base[b]], "delta": delta_all, "logits": logits,
            "inds": inds, "gates": gates, "aux": aux, "z": z, "counts": counts, "ortho": ortho}


def make_case(name, dtype, B, T, C, F, E, k, r, seed, prev=False, bias=False, gate_dtype=None, adapter_dtype=None):
    rng = np.random.default_rng(seed)

    def draw(shape, scale=1.0, uniform=False, dt=None):
        a = rng.uniform(0, 1, shape) if uniform else rng.standard_normal(shape) * scale
        return np.vectorize(lambda v: rnd(v, dt or dtype))(a).astype(np.float64)

    x = draw((B, T, C))
    p = {"x_k": draw((C,), uniform=True), "Wk": draw((F, C), 1 / math.sqrt(C)), "Wv": draw((C, F), 1 / math.sqrt(F)),
         "Wg": draw((E, C), 1 / math.sqrt(C), dt=gate_dtype), "A": draw((E, C, r), 1 / math.sqrt(C), dt=adapter_dtype),
         "B": draw((E, r, C), 0.02, dt=adapter_dtype)}
    xp = draw((B, C)) if prev else None
    bs = np.array([r32(v) for v in np.log(np.arange(1, E + 1, dtype=np.float64) ** -1.2 /
                                          np.sum(np.arange(1, E + 1, dtype=np.float64) ** -1.2))]) if bias else None
    res = forward(x.tolist(), {k2: v.tolist() for k2, v in p.items()}, k, dtype,
                  None if xp is None else xp.tolist(), None if bs is None else bs.tolist(), gate_dtype, adapter_dtype)
    arrays = {f"in_{k2}": v.astype(np.float32) for k2, v in p.items()}
    arrays["in_x"] = x.astype(np.float32)
    if xp is not None:
        arrays["in_x_prev"] = xp.astype(np.float32)
    if bs is not None:
        arrays["in_bias"] = bs.astype(np.float32)
    for k2 in ("out", "base", "delta", "logits", "gates"):
        arrays[f"out_{k2}"] = np.array(res[k2], np.float32)
    arrays["out_inds"] = np.array(res["inds"], np.int32)
    arrays["out_counts"] = np.array(res["counts"], np.int64)
    arrays["out_aux"] = np.array(res["aux"], np.float64)
    arrays["out_z"] = np.array(res["z"], np.float64)
    arrays["out_ortho"] = np.array(res["ortho"], np.float64)
    arrays["meta"] = np.array([B, T, C, F, E, k, r], np.int64)
    arrays["dtype"] = np.array(dtype)
    arrays["gate_dtype"] = np.array(gate_dtype or dtype)
    arrays["adapter_dtype"] = np.array(adapter_dtype or dtype)
    np.savez_compressed(OUT / f"{name}.npz", **arrays)
    print(f"wrote {name}.npz")


CASES = [
    ("kat_f32_e4_top1", "f32", 2, 3, 64, 16, 4, 1, 2, 11, False, False),
    ("kat_f16_e4_top2", "f16", 2, 3, 64, 16, 4, 2, 2, 12, False, False),
    ("kat_bf16_e8_top2_prev", "bf16", 2, 2, 64, 8, 8, 2, 3, 13, True, False),
    ("kat_f16_e6_top4_bias", "f16", 1, 4, 128, 8, 6, 4, 2, 14, False, True),
    # the reference's fine-tune layer: fp16 base (convert.py) with fp32 gate and adapters (moe.py:47, 124-125)
    ("kat_f16base_f32adapters_e4_top2", "f16", 2, 3, 64, 16, 4, 2, 2, 15, False, False, "f32", "f32"),
]

if __name__ == "__main__":
    import sys
    for c in CASES:
        if len(sys.argv) == 1 or c[0] in sys.argv[1:]:
            make_case(*c)
