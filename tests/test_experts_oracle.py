"""Pins of the full-expert (MoE_CMix) oracle on the CPU: one expert with
top-1 is the plain ChannelMix; the routed-rows evaluation equals the
reference's dense masked loop exactly; an expert whose value weights are zero
contributes nothing to the tokens it serves; x_k = 0 reduces the token shift
away."""
from __future__ import annotations

import numpy as np

from oracle import moe_oracle as O


def _params(rng, E, C, F, dtype):
    r = lambda a: O.round_to(a, dtype)
    return {"x_k": r(rng.uniform(0, 1, (E, C))), "Wk": r(rng.standard_normal((E, F, C)) / np.sqrt(C)),
            "Wv": r(rng.standard_normal((E, C, F)) / np.sqrt(F)), "Wg": r(rng.standard_normal((E, C)) / np.sqrt(C))}


def test_single_expert_is_the_channel_mix():
    rng = np.random.default_rng(1)
    p = _params(rng, 1, 64, 128, "f16")
    x = O.round_to(rng.standard_normal((2, 9, 64)), "f16")
    out, aux, z = O.experts_forward(x, p, 1, "f16")
    base = O.cmix_base(x, p["x_k"][0], p["Wk"][0], p["Wv"][0], "f16")
    assert np.array_equal(out, base)
    assert abs(aux - 1.0) < 1e-12  # one expert: f = 1, p = 1, E = 1


def test_routed_rows_equal_dense_loop():
    rng = np.random.default_rng(2)
    E, C, F, k = 5, 64, 128, 2
    for dtype in ("f32", "f16", "bf16"):
        p = _params(rng, E, C, F, dtype)
        x = O.round_to(rng.standard_normal((3, 7, C)), dtype)
        xp = O.round_to(rng.standard_normal((3, C)), dtype)
        parts = O.experts_forward(x, p, k, dtype, x_prev=xp, return_parts=True)
        rows = np.arange(21)
        got = O.experts_rows(x, p, k, dtype, rows, parts, x_prev=xp)
        assert np.array_equal(got, parts["out"].reshape(-1, C)), dtype


def test_zero_value_expert_contributes_nothing():
    rng = np.random.default_rng(3)
    E, C, F, k = 4, 64, 128, 1
    p = _params(rng, E, C, F, "f32")
    p["Wv"][2] = 0
    x = rng.standard_normal((1, 16, C)).astype(np.float32)
    parts = O.experts_forward(x, p, k, "f32", return_parts=True)
    hit = parts["inds"][:, 0] == 2
    assert np.all(parts["out"].reshape(-1, C)[hit] == 0)
    assert np.any(parts["out"].reshape(-1, C)[~hit] != 0)


def test_zero_mix_uses_x_alone():
    rng = np.random.default_rng(4)
    E, C, F, k = 3, 64, 128, 2
    p = _params(rng, E, C, F, "f32")
    p["x_k"][:] = 0
    x = rng.standard_normal((2, 5, C)).astype(np.float32)
    parts = O.experts_forward(x, p, k, "f32", return_parts=True)
    # with x_k = 0 each expert sees x itself: evaluate every row as a 1-token sequence
    rows = np.arange(10)
    got = O.experts_rows(x.reshape(10, 1, C), p, k, "f32", rows, parts)
    assert np.array_equal(got, parts["out"].reshape(-1, C))
