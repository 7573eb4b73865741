"""The oracle's dense GEGLU (Array::geglu, native/ffi/mlx_bridge.cpp:764-774:
0.5g * (1 + tanh(0.7978845608 * (g + 0.044715 * g^3))) * u, a compiled MLX
expression evaluated on float16 arrays with f16 constants) pinned three ways:
* the reference's own unit test (native/src/array.rs:3114-3118): gate [0, 1],
  up [2, 3] give [0, 2.5236 +- 0.001];
* numpy's float16 arithmetic evaluating the same staged expression, with pow
  and tanh taken in float64 and rounded once to f16: bit-exact for every
  finite f16 gate;
* the exact tanh-GELU in float64: for every finite gate the f16 roundings keep
  the error below 2^-10 |g| + 2^-24 (a dropped cube term or a wrong constant
  exceeds it; the erf GELU stays within it, 2e-4 relative, as it does within
  the unit test's 0.001 -- the tanh form is the one mlx_bridge.cpp:770-772
  writes).
Apple's half-precision pow and tanh are not available here; the oracle rounds
them once from binary64, and bit parity with the engine on its GPU is not
claimed beyond the unit test above.
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
    with np.errstate(over="ignore", invalid="ignore"):
        gd = g.astype(np.float64)
        cube = (gd * gd * gd).astype(np.float16)
        t = g + np.float16(0.044715) * cube
        inner = np.float16(0.7978845608028654) * t
        th = np.tanh(inner.astype(np.float64)).astype(np.float16)
        gelu = (np.float16(0.5) * g) * (np.float16(1) + th)
        return gelu * u


def exact(g, u=1.0):
    gd = np.asarray(g, np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        return 0.5 * gd * (1.0 + np.tanh(0.7978845608028654 * (gd + 0.044715 * gd ** 3))) * u


def test_reference_unit_test_values():
    out = oracle.geglu(np.array([0, 1], np.float16), np.array([2, 3], np.float16))
    assert out[0] == 0
    assert abs(float(out[1]) - 2.5236) < 1e-3


def test_matches_numpy_f16_staging_for_every_gate():
    g = all_finite_f16()
    for u in (np.float16(1), np.float16(-0.75), np.float16(3.5)):
        uu = np.full_like(g, u)
        got = oracle.geglu(g, uu)
        want = numpy_staged(g, uu)
        same = (got.view(np.uint16) == want.view(np.uint16)) | (np.isnan(got) & np.isnan(want))
        assert same.all(), (g[~same][:5], got[~same][:5], want[~same][:5])


def test_close_to_the_exact_tanh_gelu():
    g = all_finite_f16()
    got = oracle.geglu(g, np.ones_like(g)).astype(np.float64)
    want = exact(g)
    ok = np.isfinite(want) & (np.abs(want) < 65000)
    err = np.abs(got[ok] - want[ok])
    assert (err <= np.abs(g[ok].astype(np.float64)) * 2.0 ** -10 + 2.0 ** -24).all()


@pytest.mark.parametrize("wrong", ["no_cube", "half_constant"])
def test_bound_detects_wrong_formulas(wrong):
    g = all_finite_f16()
    gd = g.astype(np.float64)
    if wrong == "no_cube":
        val = 0.5 * gd * (1.0 + np.tanh(0.7978845608028654 * gd))
    else:
        val = 0.5 * gd * (1.0 + np.tanh(0.5 * (gd + 0.044715 * gd ** 3)))
    want = exact(g)
    ok = np.isfinite(want) & (np.abs(want) < 65000) & np.isfinite(val)
    err = np.abs(val[ok] - want[ok])
    assert (err > np.abs(gd[ok]) * 2.0 ** -10 + 2.0 ** -24).any()


def test_large_gates_saturate_exactly():
    # tanh rounds to +-1 in f16: gelu(g) = g for large positive g, and the
    # 1 + tanh cancellation gives exactly zero for large negative g
    g = np.array([8, 16, 100, 1000], np.float16)
    np.testing.assert_array_equal(oracle.geglu(g, np.ones_like(g)), g)
    out = oracle.geglu(-g, np.ones_like(g))
    assert (out == 0).all()
