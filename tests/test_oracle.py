"""Pins for the CPU oracle (oracle/moe_oracle.py), each chosen so that a
plausible mistake (a dropped term, a wrong sign or index, a transposed
operand, a wrong rounding point) fails at least one of them:

* rounding helpers against torch's and numpy's casts;
* router logits against a pure-Python loop of the exact definition and
  against exact rational sums; top-k against a brute-force sort and ties;
* gates, z and aux against closed forms;
* dispatch against a brute-force stable sort and its invariants;
* base ChannelMix against pure-Python loops and its special cases
  (x_k = 0, x_k = 1, sequence start, decode equivalence);
* expert adapters against B = 0, identical experts and the sparse form;
* ortho loss against orthogonal and identical column spaces;
* everything against the brute-force known-answer fixtures in tests/golden/.
"""
from __future__ import annotations

import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import moe_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"
ULP = {"f32": 2.0 ** -23, "f16": 2.0 ** -10, "bf16": 2.0 ** -7}


def rng(seed=0):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------------------
# rounding
# ---------------------------------------------------------------------------

def test_bf16_round_matches_torch():
    import torch
    a = np.concatenate([rng(1).standard_normal(100000).astype(np.float32) * 10.0 ** rng(2).integers(-30, 30, 100000),
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 65504.0, 3.4e38, -3.4e38, np.inf, -np.inf],
                                 np.float32)]).astype(np.float32)
    ref = torch.from_numpy(a).to(torch.bfloat16).to(torch.float32).numpy()
    got = O.bf16_round(a)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_round_to_f16_and_f32():
    a = rng(3).standard_normal(1000).astype(np.float32)
    assert np.array_equal(O.round_to(a, "f16"), a.astype(np.float16).astype(np.float32))
    assert np.array_equal(O.round_to(a, "f32"), a)
    with pytest.raises(ValueError):
        O.round_to(a, "f8")


# ---------------------------------------------------------------------------
# router
# ---------------------------------------------------------------------------

def _logit_loop(x, w):
    """The logit definition as scalar Python arithmetic (floats are fp64)."""
    tot = 0.0
    for q in range(len(x) // 64):
        acc = 0.0
        for j in range(64):
            acc = acc + float(x[64 * q + j]) * float(w[64 * q + j])
        tot = tot + acc
    return np.float32(tot)


def test_router_logits_match_scalar_loop():
    x = O.round_to(rng(4).standard_normal((5, 192)), "f16")
    w = O.round_to(rng(5).standard_normal((3, 192)) / 14, "f16")
    got = O.router_logits(x, w)
    for t in range(5):
        for e in range(3):
            assert got[t, e].view(np.uint32) == _logit_loop(x[t], w[e]).view(np.uint32)


def _r32_exact(q):
    """Exact rational -> nearest fp32 (ties to even) by integer arithmetic."""
    if q == 0:
        return 0.0
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 23)
    m = a / ulp
    fl = m.numerator // m.denominator
    rem = m - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return sign * float(fl * ulp)


def _logit_loop_f32(x, w):
    """The fp32-accumulator logit definition as exact rational arithmetic:
    each FMA is the exact value rounded once to fp32; chunks summed in fp64."""
    tot = 0.0
    for q in range(len(x) // 64):
        acc = 0.0
        for j in range(64):
            acc = _r32_exact(Fraction(acc) + Fraction(float(x[64 * q + j])) * Fraction(float(w[64 * q + j])))
        tot = tot + acc
    return np.float32(tot)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_router_logits_f32_accumulator_matches_exact_fma_loop(dtype):
    x = O.round_to(rng(31).standard_normal((4, 128)) * 3, dtype)
    w = O.round_to(rng(32).standard_normal((3, 128)) / 5, dtype)
    x[0, :64] = O.round_to(np.linspace(-1e3, 1e3, 64), dtype)      # wide dynamic range in one chunk
    w[0, :64] = O.round_to(np.geomspace(1e-4, 10, 64), dtype)
    got = O.router_logits(x, w, acc="f32")
    for t in range(4):
        for e in range(3):
            assert got[t, e].view(np.uint32) == _logit_loop_f32(x[t], w[e]).view(np.uint32), (t, e)
    # the layer's dtype picks the accumulator
    assert O.logit_acc("f16") == O.logit_acc("bf16") == "f32" and O.logit_acc("f32") == "f64"
    r = O.router(x, w, 2, dtype)
    assert np.array_equal(r["logits"].view(np.uint32), got.view(np.uint32))


def test_router_logits_f32_accumulator_error_bound():
    # |fp32 chunk sum - exact| <= 64·u·Σ|x·w| per chunk (u = 2^-24), plus the final fp32 rounding
    x = O.round_to(rng(33).standard_normal((16, 256)), "f16")
    w = O.round_to(rng(34).standard_normal((5, 256)) / 16, "f16")
    got = O.router_logits(x, w, acc="f32").astype(np.float64)
    for t in range(16):
        for e in range(5):
            exact = float(sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(x[t], w[e])))
            bound = 64 * 2.0 ** -24 * float(np.sum(np.abs(x[t].astype(np.float64) * w[e]))) + abs(exact) * 2.0 ** -24
            assert abs(got[t, e] - exact) <= bound


def test_router_logits_within_one_ulp_of_exact():
    x = rng(6).standard_normal((20, 128)).astype(np.float32)
    w = (rng(7).standard_normal((4, 128)) / 11).astype(np.float32)
    got = O.router_logits(x, w)
    for t in range(20):
        for e in range(4):
            exact = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(x[t], w[e]))
            assert abs(float(got[t, e]) - float(exact)) <= np.spacing(np.float32(abs(float(exact))))


def test_router_logits_one_hot_and_bias():
    E, C = 4, 64
    w = O.round_to(rng(8).standard_normal((E, C)), "f16")
    x = np.zeros((C, C), np.float32)
    x[np.arange(C), np.arange(C)] = 1.0
    assert np.array_equal(O.router_logits(x, w), w.T)          # transposed operand would fail
    b = np.array([0.5, -1.0, 0.0, 2.0], np.float32)
    assert np.array_equal(O.router_logits(x, w, b), (w.T + b).astype(np.float32))
    with pytest.raises(ValueError):
        O.router_logits(np.zeros((2, 65), np.float32), np.zeros((2, 65), np.float32))


def test_topk_brute_force_and_ties():
    lg = O.round_to(rng(9).standard_normal((300, 7)), "bf16")  # bf16 grid: many ties
    lg[:20] = 1.0                                               # all-equal rows
    for k in (1, 2, 3, 7):
        got = O.topk_canonical(lg, k)
        for t in range(lg.shape[0]):
            ref = sorted(range(7), key=lambda e: (-lg[t, e], e))[:k]
            assert got[t].tolist() == ref
            unsel = np.setdiff1d(np.arange(7), got[t])
            if unsel.size:
                assert lg[t, got[t]].min() >= lg[t, unsel].max()
    assert np.array_equal(O.topk_canonical(lg, 1)[:, 0], np.argmax(lg, axis=1))
    assert O.topk_canonical(lg[:1], 3)[0].tolist() == [0, 1, 2]  # ties to the lower id


def test_gates_closed_forms():
    x = O.round_to(rng(10).standard_normal((64, 128)), "f32")
    w = O.round_to(rng(11).standard_normal((6, 128)) / 11, "f32")
    r1 = O.router(x, w, 1, "f32")
    assert np.all(r1["gates"] == 1.0)
    r2 = O.router(x, w, 2, "f32")
    l = r2["logits"]
    l0 = np.take_along_axis(l, r2["inds"][:, :1], 1)[:, 0].astype(np.float64)
    l1 = np.take_along_axis(l, r2["inds"][:, 1:2], 1)[:, 0].astype(np.float64)
    g0 = 1.0 / (1.0 + np.exp(l1 - l0))
    assert np.allclose(r2["gates"][:, 0], g0, rtol=2e-7, atol=0)
    assert np.allclose(r2["gates"].sum(1), 1.0, atol=2e-7)
    assert np.all(r2["gates"][:, 0] >= r2["gates"][:, 1])


def test_z_loss_closed_form():
    E = 5
    x = np.zeros((10, 64), np.float32)
    w = np.zeros((E, 64), np.float32)
    r = O.router(x, w, 2, "f32")
    assert math.isclose(r["z"], math.log(E) ** 2, rel_tol=1e-6)
    x = O.round_to(rng(12).standard_normal((40, 64)), "f32")
    w = O.round_to(rng(13).standard_normal((E, 64)) / 8, "f32")
    r = O.router(x, w, 2, "f32")
    ref = np.mean([math.log(sum(math.exp(float(v)) for v in row)) ** 2 for row in r["logits"]])
    assert math.isclose(r["z"], ref, rel_tol=1e-6)


def test_aux_closed_forms():
    E = 4
    # balanced routing with uniform probabilities -> aux = 1
    N = 8
    x = np.zeros((N, 64), np.float32)
    w = np.zeros((E, 64), np.float32)
    bias = np.zeros(E, np.float32)
    r = O.router(x, w, E, "f32", bias)  # k = E: every expert chosen once per token
    assert math.isclose(r["aux"], 1.0, rel_tol=1e-7)
    # every token routes to expert 2 with near one-hot probabilities -> aux = E / k
    for k in (1, 2):
        b = np.array([0.0, 0.0, 40.0, 0.0], np.float32)
        r = O.router(x, w, k, "f32", b)
        assert np.all(r["inds"][:, 0] == 2)
        assert math.isclose(r["aux"], E / k + (0 if k == 1 else E * 0.5 * 0.0), rel_tol=1e-6) or k == 2
        if k == 2:  # f = (1/2 for e=2, 1/2 for e=0), p = (~0, ~0, ~1, ~0) -> aux = E/2
            assert math.isclose(r["aux"], E / 2, rel_tol=1e-6)


# ---------------------------------------------------------------------------
# dispatch
# ---------------------------------------------------------------------------

def test_dispatch_brute_force():
    E = 6
    inds = rng(14).integers(0, E, size=(257, 3)).astype(np.int32)
    perm, inv, offs = O.dispatch(inds, E)
    flat = inds.reshape(-1).tolist()
    ref = sorted(range(len(flat)), key=lambda a: (flat[a], a))
    assert perm.tolist() == ref
    assert sorted(perm.tolist()) == list(range(len(flat)))
    assert np.all(np.diff(np.array(flat)[perm]) >= 0)
    assert np.array_equal(inv[perm], np.arange(len(flat)))
    counts = [flat.count(e) for e in range(E)]
    assert offs.tolist() == [0] + np.cumsum(counts).tolist()
    for e in range(E):
        seg = perm[offs[e]:offs[e + 1]]
        assert np.all(np.diff(seg) > 0)            # stable: ascending assignment ids
        assert all(flat[a] == e for a in seg)


# ---------------------------------------------------------------------------
# base ChannelMix
# ---------------------------------------------------------------------------

def _r(v, dtype):
    """Scalar rounding to the layer dtype."""
    return float(np.asarray(O.round_to(v, dtype)).reshape(-1)[0])


def _base_loop(x, mu, Wk, Wv, dtype, x_prev=None):
    B, T, C = x.shape
    out = np.zeros_like(x)
    for b in range(B):
        for t in range(T):
            prev = x[b, t - 1] if t > 0 else (x_prev[b] if x_prev is not None else np.zeros(C, np.float32))
            kin = [_r(x[b, t, c] + _r(_r(prev[c] - x[b, t, c], dtype) * mu[c], dtype), dtype) for c in range(C)]
            h = []
            for f in range(Wk.shape[0]):
                v = _r(float(sum(Fraction(float(a)) * Fraction(float(b2)) for a, b2 in zip(kin, Wk[f]))), dtype)
                v = max(v, 0.0)
                h.append(_r(v * v, dtype))
            for c in range(C):
                out[b, t, c] = _r(float(sum(Fraction(a) * Fraction(float(b2)) for a, b2 in zip(h, Wv[c]))), dtype)
    return out


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_base_against_loops(dtype):
    g = rng(15)
    x = O.round_to(g.standard_normal((2, 3, 8)), dtype)
    mu = O.round_to(g.uniform(0, 1, 8), dtype)
    Wk = O.round_to(g.standard_normal((6, 8)) / 3, dtype)
    Wv = O.round_to(g.standard_normal((8, 6)) / 2.5, dtype)
    xp = O.round_to(g.standard_normal((2, 8)), dtype)
    for prev in (None, xp):
        got = O.cmix_base(x, mu, Wk, Wv, dtype, prev)
        ref = _base_loop(x, mu, Wk, Wv, dtype, prev)
        assert np.max(np.abs(got - ref)) <= ULP[dtype] * np.max(np.abs(ref)) * 2


def test_base_special_cases():
    g = rng(16)
    x = O.round_to(g.standard_normal((2, 5, 16)), "f32")
    Wk = O.round_to(g.standard_normal((24, 16)) / 4, "f32")
    Wv = O.round_to(g.standard_normal((16, 24)) / 5, "f32")
    # x_k = 0: no shift at all
    ref0 = np.maximum(x.astype(np.float64) @ Wk.T, 0) ** 2 @ Wv.T
    assert np.allclose(O.cmix_base(x, np.zeros(16, np.float32), Wk, Wv, "f32"), ref0, rtol=1e-5, atol=1e-5)
    # x_k = 1: the previous token only; row 0 of each sequence sees zeros
    prev = O.time_shift(x)
    assert np.all(prev[:, 0] == 0) and np.array_equal(prev[:, 1:], x[:, :-1])
    ref1 = np.maximum(prev.astype(np.float64) @ Wk.T, 0) ** 2 @ Wv.T
    assert np.allclose(O.cmix_base(x, np.ones(16, np.float32), Wk, Wv, "f32"), ref1, rtol=1e-5, atol=1e-5)
    # T = 1 without state: xk = x * (1 - x_k)
    mu = O.round_to(g.uniform(0, 1, 16), "f32")
    x1 = x[:, :1]
    ref2 = np.maximum((x1 * (1 - mu)).astype(np.float64) @ Wk.T, 0) ** 2 @ Wv.T
    assert np.allclose(O.cmix_base(x1, mu, Wk, Wv, "f32"), ref2, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_decode_equivalence(dtype):
    """decode(x, x_prev) == forward([x_prev, x])[:, 1] (model.py:498-506 vs 259-263)."""
    g = rng(17)
    x = O.round_to(g.standard_normal((4, 64)), dtype)
    xp = O.round_to(g.standard_normal((4, 64)), dtype)
    mu = O.round_to(g.uniform(0, 1, 64), dtype)
    Wk = O.round_to(g.standard_normal((128, 64)) / 8, dtype)
    Wv = O.round_to(g.standard_normal((64, 128)) / 11, dtype)
    out, state = O.cmix_decode(x, xp, mu, Wk, Wv, dtype)
    seq = np.stack([xp, x], axis=1)
    ref = O.cmix_base(seq, mu, Wk, Wv, dtype)[:, 1]
    assert np.array_equal(out, ref)
    assert np.array_equal(state, x)
    assert np.array_equal(O.cmix_base(x[:, None], mu, Wk, Wv, dtype, x_prev=xp)[:, 0], ref)


# ---------------------------------------------------------------------------
# expert adapters
# ---------------------------------------------------------------------------

def _layer(dtype, N=40, C=64, E=5, k=2, r=3, seed=18):
    g = rng(seed)
    x = O.round_to(g.standard_normal((N, C)), dtype)
    A = O.round_to(g.standard_normal((E, C, r)) / 8, dtype)
    B = O.round_to(g.standard_normal((E, r, C)) * 0.02, dtype)
    Wg = O.round_to(g.standard_normal((E, C)) / 8, dtype)
    r_ = O.router(x, Wg, k, dtype)
    return x, A, B, r_


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_lora_zero_B_gives_zero_delta(dtype):
    x, A, B, r = _layer(dtype)
    d = O.lora_delta_dense(x, A, np.zeros_like(B), r["inds"], r["gates"], dtype)
    assert np.all(d == 0)


def test_lora_identical_experts():
    x, A, B, r = _layer("f32", k=3)
    A[:] = A[0]
    B[:] = B[0]
    d = O.lora_delta_dense(x, A, B, r["inds"], r["gates"], "f32")
    ref = (x.astype(np.float64) @ A[0]) @ B[0]
    assert np.allclose(d, ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_lora_sparse_equals_dense(dtype):
    for k in (1, 2, 4):
        x, A, B, r = _layer(dtype, k=k)
        dd = O.lora_delta_dense(x, A, B, r["inds"], r["gates"], dtype)
        ds = O.lora_delta_sparse(x, A, B, r["inds"], r["gates"], dtype)
        assert np.array_equal(dd, ds)


def test_lora_brute_force_tiny():
    x, A, B, r = _layer("f32", N=6, C=64, E=3, k=2, r=2)
    d = O.lora_delta_dense(x, A, B, r["inds"], r["gates"], "f32")
    for t in range(6):
        ref = np.zeros(64)
        for s in range(2):
            e = r["inds"][t, s]
            u = [sum(float(x[t, c]) * float(A[e, c, j]) for c in range(64)) for j in range(2)]
            ref += float(r["gates"][t, s]) * np.array([sum(u[j] * float(B[e, j, c]) for j in range(2))
                                                       for c in range(64)])
        assert np.allclose(d[t], ref, rtol=1e-5, atol=1e-7)


# ---------------------------------------------------------------------------
# orthogonality loss
# ---------------------------------------------------------------------------

def test_ortho_closed_forms():
    E, C, r = 4, 64, 2
    A = np.zeros((E, C, r), np.float32)
    for e in range(E):
        for j in range(r):
            A[e, e * r + j, j] = 1.0      # disjoint coordinate blocks: orthogonal column spaces
    assert O.ortho_loss(A, "f32") == 0.0
    A2 = np.zeros((E, C, r), np.float32)
    A2[:, 0, 0] = 1.0                     # every expert shares one unit column
    assert O.ortho_loss(A2, "f32") == E * (E - 1) / 2
    g = rng(19).standard_normal((3, 64, 2)).astype(np.float32)
    ref = sum(float(np.sum((g[i].T.astype(np.float64) @ g[j]) ** 2)) for i in range(3) for j in range(i + 1, 3))
    assert math.isclose(O.ortho_loss(g, "f32"), ref, rel_tol=1e-5)


# ---------------------------------------------------------------------------
# known-answer fixtures (tests/golden/make_fixtures.py)
# ---------------------------------------------------------------------------

FIXTURES = sorted(GOLDEN.glob("kat_*.npz"))


def test_fixtures_present():
    assert len(FIXTURES) >= 5


@pytest.mark.parametrize("path", FIXTURES, ids=[p.stem for p in FIXTURES])
def test_oracle_matches_fixture(path):
    z = np.load(path)
    dtype = str(z["dtype"])
    gdt, adt = str(z["gate_dtype"]), str(z["adapter_dtype"])
    ad = O.promote(dtype, adt)  # the delta's and the output's dtype
    B, T, C, F, E, k, r = (int(v) for v in z["meta"])
    p = {"x_k": z["in_x_k"], "Wk": z["in_Wk"], "Wv": z["in_Wv"], "Wg": z["in_Wg"], "A": z["in_A"], "B": z["in_B"]}
    xp = z["in_x_prev"] if "in_x_prev" in z else None
    bias = z["in_bias"] if "in_bias" in z else None
    parts = O.moe_forward(z["in_x"], p, k, dtype, x_prev=xp, bias=bias, return_parts=True, gate_dtype=gdt,
                          adapter_dtype=adt)
    assert np.array_equal(parts["logits"].view(np.uint32), z["out_logits"].view(np.uint32))
    assert np.array_equal(parts["inds"], z["out_inds"])
    assert np.array_equal(parts["counts"], z["out_counts"])
    assert np.max(np.abs(parts["gates"] - z["out_gates"])) <= ULP[dtype]
    assert math.isclose(parts["aux"], float(z["out_aux"]), rel_tol=1e-6)
    assert math.isclose(parts["z"], float(z["out_z"]), rel_tol=1e-6)
    scale = float(np.max(np.abs(z["out_out"])))
    assert np.max(np.abs(parts["base"] - z["out_base"])) <= 2 * ULP[dtype] * scale
    assert np.max(np.abs(parts["delta"] - z["out_delta"])) <= 2 * ULP[ad] * scale
    # out = round_ad(base + delta): the base's dtype bounds its error
    assert np.max(np.abs(parts["out"].reshape(-1, C) - z["out_out"])) <= 2 * ULP[dtype] * scale
    assert math.isclose(O.ortho_loss(p["A"], adt), float(z["out_ortho"]), rel_tol=4 * ULP[adt], abs_tol=1e-9)


# ---------------------------------------------------------------------------
# planted mistakes: the pins above must catch a broken oracle
# ---------------------------------------------------------------------------

def test_planted_mistakes_are_caught(monkeypatch):
    path = FIXTURES[1]
    z = np.load(path)
    dtype = str(z["dtype"])
    k = int(z["meta"][5])
    p = {"x_k": z["in_x_k"], "Wk": z["in_Wk"], "Wv": z["in_Wv"], "Wg": z["in_Wg"], "A": z["in_A"], "B": z["in_B"]}

    def max_err():
        parts = O.moe_forward(z["in_x"], p, k, dtype, return_parts=True)
        return float(np.max(np.abs(parts["out"].reshape(z["out_out"].shape) - z["out_out"])))

    ok = max_err()
    orig_shift = O.time_shift
    monkeypatch.setattr(O, "time_shift", lambda x, xp=None: np.roll(orig_shift(x, xp), -1, axis=1))
    assert max_err() > 100 * max(ok, 1e-6)           # shift in the wrong direction
    monkeypatch.setattr(O, "time_shift", orig_shift)
    orig_topk = O.topk_canonical
    monkeypatch.setattr(O, "topk_canonical", lambda l, kk: np.argsort(l, axis=-1, kind="stable")[..., :kk]
                        .astype(np.int32))
    assert max_err() > 10 * max(ok, 1e-6)            # smallest instead of largest logits
    monkeypatch.setattr(O, "topk_canonical", orig_topk)
    p["A"] = p["A"][:, ::-1].copy()                  # a reversed reduction axis in the adapter
    assert max_err() > 10 * max(ok, 1e-6)


def test_mixed_fixture_pins_mlx_promotion():
    """The fp16-base / fp32-adapter fixture catches an oracle that drops MLX
    promotion: computing the delta in fp16 (the old all-one-dtype rule), or
    the logits with the fp16 layer's fp32 chunk accumulator instead of the
    fp64 one an fp32 gate calls for."""
    z = np.load(GOLDEN / "kat_f16base_f32adapters_e4_top2.npz")
    k = int(z["meta"][5])
    C = int(z["meta"][2])
    p = {"x_k": z["in_x_k"], "Wk": z["in_Wk"], "Wv": z["in_Wv"], "Wg": z["in_Wg"], "A": z["in_A"], "B": z["in_B"]}
    scale = float(np.max(np.abs(z["out_out"])))
    good = O.moe_forward(z["in_x"], p, k, "f16", return_parts=True, gate_dtype="f32", adapter_dtype="f32")
    assert np.max(np.abs(good["delta"] - z["out_delta"])) <= 2 * ULP["f32"] * scale
    assert good["out"].dtype == np.float32 and not np.array_equal(good["out"], O.round_to(good["out"], "f16"))
    # the delta in fp16 (and out rounded to fp16) misses the fixture by far more than fp32 rounding
    bad = O.moe_forward(z["in_x"], p, k, "f16", return_parts=True, gate_dtype="f32")
    assert np.max(np.abs(bad["delta"] - z["out_delta"])) > 50 * ULP["f32"] * scale
    assert np.max(np.abs(bad["out"].reshape(-1, C) - z["out_out"])) > 50 * ULP["f32"] * scale
    # the logits with the 16-bit layer's accumulator are not the fixture's bits
    lg16 = O.router_logits(z["in_x"].reshape(-1, C), p["Wg"], acc="f32")
    assert not np.array_equal(lg16.view(np.uint32), z["out_logits"].view(np.uint32))
