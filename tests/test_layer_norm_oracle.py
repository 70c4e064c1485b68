"""Pins of the ln2 restatement (oracle/moe_oracle.py ``layer_norm``, the
Block's nn.LayerNorm in front of the ChannelMix, model.py:283, 321, and the
RNN form _layer_norm_1d, model.py:434-438) on the CPU.

* Against torch.nn.functional.layer_norm in float64 (an independent
  implementation), rounded the same way: equal in every element.
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
def test_matches_torch_float64(dtype, C):
    torch = pytest.importorskip("torch")
    x, w, b = _row_data(33, C, dtype, seed=C)
    got = O.layer_norm(x, w, b, dtype)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x.astype(np.float64)), (C,),
                                         torch.from_numpy(w.astype(np.float64)),
                                         torch.from_numpy(b.astype(np.float64)), eps=1e-5).numpy()
    assert np.array_equal(got, O.round_to(ref, dtype))


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
