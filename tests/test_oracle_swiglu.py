"""The oracle's dense SwiGLU (Array::swiglu, native/ffi/mlx_bridge.cpp:745-749:
(g * sigmoid(g)) * u evaluated on float16 arrays with MLX's Sigmoid
y = 1 / (1 + exp(-|x|)), x < 0 ? 1 - y : y) pinned three ways:
* numpy's own float16 arithmetic (each operation computed wider and rounded to
  f16) evaluating the same staged expression, with exp taken in float64 and
  rounded to f32 and then f16 (numpy's float16 exp loop is not correctly
  rounded, e.g. exp(-0.04724) comes out one f16 ulp high): bit-exact, for
  every finite f16 gate value;
* the exact value g * u / (1 + e^-g) in float64: the f16 roundings bound the
  error by 4 f16 ulp of the result plus 2^-10 |g u| (the sigmoid's absolute
  error; for g < 0 the cancellation in 1 - y makes tiny results inexact), and
  by 4 ulp alone for g >= 0 (the sigmoid of -g in its place fails the bound);
* MLX's precise_swiglu (mlx_bridge.cpp:752-758: f32 silu, f32 product, one f16
  rounding), within the same bound.
Apple's half-precision exp is not available here, so bit parity with the
engine on its GPU is not claimed; the tolerance above is what is checked.
"""

import numpy as np
import pytest

import oracle


def all_finite_f16():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    v = bits.view(np.float16)
    return v[np.isfinite(v)]


def numpy_staged(g, u):
    g = g.astype(np.float16)
    u = u.astype(np.float16)
    one = np.float16(1)
    with np.errstate(over="ignore"):
        e = np.exp(-np.abs(g).astype(np.float64)).astype(np.float32).astype(np.float16)
        y = one / (one + e)
        s = np.where(g < 0, one - y, y).astype(np.float16)
        return (g * s) * u


def ulps(a, b):
    """|a - b| in units of the f16 spacing at |b| (exact reference in f64)."""
    sp = np.spacing(np.abs(b).astype(np.float16)).astype(np.float64)
    sp = np.maximum(sp, 2.0 ** -24)
    return np.abs(a.astype(np.float64) - b) / sp


@pytest.fixture(scope="module")
def inputs():
    rng = np.random.default_rng(7)
    g = np.tile(all_finite_f16(), 3)
    u = (rng.standard_normal(g.size) * 2).astype(np.float16)
    return g, u


def test_swiglu_matches_numpy_f16_staging(inputs):
    g, u = inputs
    got = oracle.swiglu(g, u)
    ref = numpy_staged(g, u)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint16), ref[~nan].view(np.uint16))


def swiglu_bound(exact, g, u):
    """Error bound of the f16-staged form: a few f16 ulp of the result, plus
    the absolute error of the f16 sigmoid (y in [1/2, 1) is known to 2^-11, and
    1 - y for g < 0 inherits that absolute error) times |g * u|."""
    sp = np.maximum(np.spacing(np.abs(exact).astype(np.float16)).astype(np.float64), 2.0 ** -24)
    return 4.0 * sp + 2.0 * 2.0 ** -11 * np.abs(g.astype(np.float64) * u.astype(np.float64))


def test_swiglu_close_to_exact(inputs):
    g, u = inputs
    got = oracle.swiglu(g, u).astype(np.float64)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        exact = g64 * u64 / (1.0 + np.exp(-g64))
    ok = np.isfinite(exact) & (np.abs(exact) < 60000)
    err = np.abs(got[ok] - exact[ok])
    assert np.all(err <= swiglu_bound(exact[ok], g[ok], u[ok]))
    # for g >= 0 the sigmoid is near 1 and the result is a few ulp off
    pos = ok & (g >= 0)
    assert (np.abs(got[pos] - exact[pos]) / np.maximum(
        np.spacing(np.abs(exact[pos]).astype(np.float16)).astype(np.float64), 2.0 ** -24)).max() <= 4
    # the bound discriminates: sigmoid(-g) in place of sigmoid(g) breaks it
    with np.errstate(over="ignore", invalid="ignore"):
        wrong = g64 * u64 / (1.0 + np.exp(g64))
    assert not np.all(np.abs(wrong[ok] - exact[ok]) <= swiglu_bound(exact[ok], g[ok], u[ok]))


def test_swiglu_near_precise_swiglu(inputs):
    g, u = inputs
    got = oracle.swiglu(g, u).astype(np.float64)
    g32, u32 = g.astype(np.float32), u.astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        precise = ((g32 / (np.float32(1) + np.exp(-g32))) * u32).astype(np.float16).astype(np.float64)
    ok = np.isfinite(precise) & (np.abs(precise) < 60000)
    assert np.all(np.abs(got[ok] - precise[ok]) <= swiglu_bound(precise[ok], g[ok], u[ok]))


def test_swiglu_special_values():
    g = np.array([0.0, -0.0, 1.0, -1.0, 20.0, -20.0, 65504.0, -65504.0], np.float16)
    u = np.array([1.0, 1.0, 2.0, 2.0, 1.0, 1.0, 1.0, 1.0], np.float16)
    out = oracle.swiglu(g, u)
    assert out[0] == 0 and out[1] == 0
    assert out[2] == np.float16(np.float16(0.731) * 2) or abs(float(out[2]) - 1.4621) < 2e-3
    assert abs(float(out[3]) + 0.5379) < 2e-3
    assert out[4] == np.float16(20.0)  # sigmoid rounds to 1 in f16
    assert out[5] == 0 or abs(float(out[5])) < 1e-6  # -20 * 2e-9: underflows to -0
    assert out[6] == np.float16(65504.0)
    assert out[7] == 0
