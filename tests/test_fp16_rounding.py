"""fp16 arithmetic the kernels run packed (v_pk_add/mul/max_f16) against the
oracle's rounding points (each op in fp32, then rounded to fp16).

The token-shift mix (model.py:260-261) and relu² (model.py:262) round after
every op on fp16 arrays.  The kernels compute those ops in packed fp16, one
IEEE rounding each; the oracle computes each op in fp32 and rounds the result
to fp16.  These agree when the fp32 result either is exact (a product or
difference of two fp16 values) or cannot land on an fp16 rounding midpoint it
was not already on (a sum of two fp16 values).  Checked here against the
exact result rounded once (float64 holds every fp16 sum and product exactly).
"""
import numpy as np

ALL_F16 = np.arange(65536, dtype=np.uint16).view(np.float16)
ALL_F16 = ALL_F16[np.isfinite(ALL_F16)]


def _check(op, rng, n_b):
    a64 = ALL_F16.astype(np.float64)
    a32 = ALL_F16.astype(np.float32)
    specials = np.float16([2 ** -24, -2 ** -24, 2 ** -14, -2 ** -14, 65504, -65504, 1.0, -1.0, 0.5, 2 ** -13, 3.0e-5])
    bs = np.concatenate([ALL_F16[rng.integers(0, ALL_F16.size, n_b)], specials])
    for b in bs:
        with np.errstate(over="ignore", invalid="ignore"):
            exact = op(a64, np.float64(b))
            single = exact.astype(np.float16)
            via32 = op(a32, np.float32(b)).astype(np.float16)
        finite = np.isfinite(single.astype(np.float64))
        mism = (single.view(np.uint16) != via32.view(np.uint16)) & finite
        assert not mism.any(), f"b={b!r}: {int(mism.sum())} mismatches, first a={ALL_F16[np.argmax(mism)]!r}"


def test_fp16_add_sub_single_rounding_equals_fp32_path():
    rng = np.random.default_rng(11)
    _check(np.add, rng, 120)
    _check(np.subtract, rng, 120)


def test_fp16_mul_single_rounding_equals_fp32_path():
    rng = np.random.default_rng(12)
    _check(np.multiply, rng, 120)


def test_relu_square_packed_equals_fp32_path():
    # relu²: round(acc) to fp16, max with 0, square with one rounding
    rng = np.random.default_rng(13)
    acc = np.concatenate([rng.standard_normal(200000).astype(np.float32) * s for s in (1e-4, 1e-2, 1.0, 30.0)])
    h = acc.astype(np.float16)
    z = np.maximum(h, np.float16(0))
    packed = (z.astype(np.float64) * z.astype(np.float64)).astype(np.float16)      # one rounding of the exact square
    with np.errstate(over="ignore"):
        via32 = (np.maximum(h.astype(np.float32), 0) ** 2).astype(np.float16)     # the oracle's form
    assert np.array_equal(packed.view(np.uint16), via32.view(np.uint16))
