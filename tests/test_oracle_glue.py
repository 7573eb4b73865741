"""The oracle's engine glue (mode 1) pinned as an exact composition.

The engine's input prologue (native/src/linear.rs:847-865) is
x.astype(F16) * suh in f16, then MLX's hadamard_transform with scale
1/sqrt(128) in its f16-staged schedule (exl3.metal:154-170); the output
epilogue (linear.rs:984-997) is sum(splits).astype(F16), the same staged
transform, * svh in f16, then astype(x.dtype).  Each part is pinned on its
own elsewhere (h128_staged by its rounding schedule in test_oracle.py, the
GEMV against a dense f64 product); here the oracle's prologue and mode-1
forward must equal, bit for bit, the composition of numpy float16 arithmetic
and that pinned h128_staged -- on random rows with suh != 1, on f16
subnormals and on signed zeros.  Two planted mistakes (no f16 rounding of
x * suh; an f32 Hadamard in place of the staged one) must each be caught.
"""

import numpy as np
import pytest

import oracle

IN, OUT = 512, 384


def f16_product(a16, b16):
    """IEEE f16 product: the f32 product of two f16 values is exact, so one
    rounding to f16 gives the correctly rounded result."""
    return (a16.astype(np.float32) * b16.astype(np.float32)).astype(np.float16)


def composed_prologue(x, suh, stage=oracle.h128_staged, round_xs=True):
    x16 = x.astype(np.float16)
    xs = f16_product(x16, suh) if round_xs else x16.astype(np.float32) * suh.astype(np.float32)
    return stage(np.asarray(xs, np.float32).reshape(-1, 128)).reshape(x.shape).astype(np.float16)


def composed_epilogue(yhat, svh, stage=oracle.h128_staged, round_yhat=True):
    y = yhat.astype(np.float16).astype(np.float32) if round_yhat else yhat.astype(np.float32)
    h = stage(y.reshape(-1, 128)).reshape(yhat.shape).astype(np.float16)
    return f16_product(h, svh)


def signed_scales(rng, n):
    return (rng.choice([-1.0, 1.0], n) * rng.uniform(0.5, 1.5, n)).astype(np.float16)


def special_rows(rng):
    """Rows of f16 subnormals, signed zeros and mixed magnitudes."""
    # sign bit, exponent 0, nonzero mantissa: every value a subnormal
    bits = rng.integers(1, 1024, IN) | (rng.integers(0, 2, IN) << 15)
    subnormal = bits.astype(np.uint16).view(np.float16)
    zeros = np.where(rng.random(IN) < 0.5, np.float16(-0.0), np.float16(0.0)).astype(np.float16)
    mixed = (rng.standard_normal(IN) * np.exp2(rng.integers(-20, 8, IN))).astype(np.float16)
    one_hot = np.zeros(IN, np.float16)
    one_hot[rng.integers(0, IN)] = np.float16(-1.0)
    return np.stack([subnormal, zeros, mixed, one_hot])


@pytest.fixture(scope="module")
def case():
    rng = np.random.default_rng(2024)
    x = np.concatenate([rng.standard_normal((6, IN)).astype(np.float16), special_rows(rng)])
    tr = rng.integers(0, 65536, (IN // 16, OUT // 16, 64), dtype=np.uint16)
    return x, tr, signed_scales(rng, IN), signed_scales(rng, OUT)


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float16).view(np.uint16),
                          np.asarray(b, np.float16).view(np.uint16))


def test_prologue_is_the_f16_composition(case):
    x, _, suh, _ = case
    assert same_bits(oracle.prologue(x, suh), composed_prologue(x, suh))


def test_prologue_keeps_signed_zeros_and_subnormal_products(case):
    x, _, suh, _ = case
    xh = oracle.prologue(x, suh)
    # an all-zero block transforms to zeros; the sign of each is the staged sum's
    zero_row = composed_prologue(x[7:8], suh)
    assert same_bits(xh[7:8], zero_row)
    assert (xh[7] == 0).all()
    # subnormal inputs times scales in [0.5, 1.5) stay representable: nonzero
    assert (xh[6] != 0).any()


@pytest.mark.parametrize("dtype", [np.float32, "bf16"])
def test_prologue_casts_wider_activations_to_f16_first(case, dtype):
    x, _, suh, _ = case
    rng = np.random.default_rng(7)
    wide = x.astype(np.float32) + rng.standard_normal(x.shape).astype(np.float32) * 1e-3
    if dtype == "bf16":
        bits = (wide.view(np.uint32) >> 16).astype(np.uint16)
        wide = (bits.astype(np.uint32) << 16).view(np.float32)
        ours = oracle.lib()
        out = np.empty(wide.size, np.uint16)
        rc = ours.exl3o_prologue(np.ascontiguousarray(bits).ctypes.data, 12, wide.shape[0], IN,
                                 suh.view(np.uint16), out)
        assert rc == 0
        got = out.view(np.float16).reshape(wide.shape)
    else:
        got = oracle.prologue(wide, suh)
    assert same_bits(got, composed_prologue(wide, suh))


def test_mode1_epilogue_is_the_f16_composition(case):
    x, tr, suh, svh = case
    y, yhat = oracle.forward(x, tr, suh, svh, 4, 0, mode=1, return_yhat=True)
    assert same_bits(y, composed_epilogue(yhat, svh))


def test_mode1_forward_is_prologue_gemv_epilogue(case):
    """The whole mode-1 forward: composed prologue, the oracle's GEMV of that
    xhat (f32, ascending k; pinned against a dense f64 product elsewhere),
    composed epilogue."""
    x, tr, suh, svh = case
    xh = composed_prologue(x, suh)
    W = oracle.reconstruct_inner(tr, 4, 0, IN, OUT).astype(np.float32)
    # the GEMV's own accumulation order: tile rows ascending, rows ascending
    yhat = np.zeros((x.shape[0], OUT), np.float32)
    xf = xh.astype(np.float32)
    for r in range(IN):
        yhat += xf[:, r:r + 1] * W[r:r + 1, :]
    y = oracle.forward(x, tr, suh, svh, 4, 0, mode=1)
    assert same_bits(y, composed_epilogue(yhat, svh))


def test_planted_mistakes_are_caught(case):
    x, tr, suh, svh = case
    xh = oracle.prologue(x, suh)
    # 1. x * suh left in f32 (no f16 rounding before the Hadamard)
    assert not same_bits(xh, composed_prologue(x, suh, round_xs=False))
    # 2. the MLX f32 Hadamard (pinned to MLX's f32 fixture) in place of the staged one
    f32_stage = lambda v: oracle.h128_f32(v)  # noqa: E731
    assert not same_bits(xh, composed_prologue(x, suh, stage=f32_stage))
    y, yhat = oracle.forward(x, tr, suh, svh, 4, 0, mode=1, return_yhat=True)
    # 3. the epilogue without the f16 rounding of the split sum
    assert not same_bits(y, composed_epilogue(yhat, svh, round_yhat=False))
    # 4. the epilogue with the f32 Hadamard
    assert not same_bits(y, composed_epilogue(yhat, svh, stage=f32_stage))
