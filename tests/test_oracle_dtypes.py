"""Pins the oracle's activation and output dtypes (CPU only).

Reference semantics:
* Exl3Linear::forward ends with ``y.astype(x.dtype)`` and then ``+ bias`` with
  the f16 bias (linear.rs:992-995, the checkpoint loader casts the bias to f16,
  :519-522).  MLX promotes bfloat16 + float16 to float32, float32 + float16 to
  float32 and keeps float16 + float16 in float16, so the result of bfloat16
  activations with a bias is float32.
* The SwitchGLU reads its input as ``half(x)`` (routed_inputs, moe.rs:205-206)
  and ends with ``f16 expert output * scores`` summed over top_k
  (finish_and_reduce, moe.rs:602-608): float16 scores give f16 products and an
  f16 result; float32 or bfloat16 scores promote the products and the sum to
  float32.

Each property is checked against values computed independently here with
numpy's IEEE float32 arithmetic and a bit-level bfloat16 rounding, from oracle
outputs whose own semantics are pinned elsewhere (the f16 path), so a missing
bf16 rounding, a sum rounded back to the activation dtype or a score product
rounded to f16 fails exactly.
"""

import numpy as np

import oracle
from mlxl3_amd import synth

F16, F32 = np.float16, np.float32


def bf16_bits(v):
    """float32 -> bfloat16 bits, round to nearest even (NaN kept quiet)."""
    b = np.asarray(v, F32).view(np.uint32).astype(np.uint64)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((b >> 16) | 0x40).astype(np.uint16), r)


def bf16_value(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(F32)


def test_bf16_rounding_helper_against_closed_forms():
    # halfway cases round to even; the largest finite bf16 stays finite
    v = np.array([1.0 + 2**-8, 1.0 + 3 * 2**-8, -2.0 - 2**-7, 3.3895314e38], F32)
    want = np.array([1.0, 1.0 + 2**-6, -2.0, 3.3895314e38], F32)
    np.testing.assert_array_equal(bf16_value(bf16_bits(v)), want)


def layer(bias):
    tr, suh, svh, b = synth.linear_layer(41, 3, 256, 256, 3, bias=bias)
    return tr, suh, svh, b


def test_linear_result_dtypes_and_bias_promotion():
    tr, suh, svh, b = layer(True)
    x32 = synth.normal(5, 1, 3 * 256).reshape(3, 256).astype(F32) * F32(1.7)
    xb = bf16_bits(x32)
    x_of_bf16 = bf16_value(xb)
    # the f16 engine result of the bf16 values, computed through f32 activations
    y16 = oracle.forward(x_of_bf16, tr, suh, svh, 3, 1).astype(F32)
    # bf16, no bias: bf16(y16)
    y_nb = oracle.forward(xb, tr, suh, svh, 3, 1, x_dtype="bf16")
    assert y_nb.dtype == np.uint16
    np.testing.assert_array_equal(y_nb, bf16_bits(y16))
    # bf16 + f16 bias: float32(bf16(y16)) + float32(bias), one f32 rounding
    y_b = oracle.forward(xb, tr, suh, svh, 3, 1, bias=b, x_dtype="bf16")
    assert y_b.dtype == F32
    want = bf16_value(bf16_bits(y16)) + b.astype(F32)
    np.testing.assert_array_equal(y_b, want)
    # and that differs from rounding the sum back to bf16 (the mistake it pins)
    assert not np.array_equal(y_b, bf16_value(bf16_bits(want)))
    # f32 + bias: y16 + bias in f32; f16 + bias: f16(y16 + bias)
    np.testing.assert_array_equal(oracle.forward(x_of_bf16, tr, suh, svh, 3, 1, bias=b),
                                  y16 + b.astype(F32))
    x16 = x32.astype(F16)
    y16h = oracle.forward(x16, tr, suh, svh, 3, 1)
    np.testing.assert_array_equal(oracle.forward(x16, tr, suh, svh, 3, 1, bias=b),
                                  (y16h.astype(F32) + b.astype(F32)).astype(F16))
    assert oracle.result_dtype(12, True) == 10 and oracle.result_dtype(12, False) == 12
    assert oracle.result_dtype(9, True) == 9 and oracle.result_dtype(10, True) == 10


def moe_case(rows=4, top_k=2, experts=5):
    bank = synth.moe_layer(8, 500, 256, 128, experts, 3)
    x = synth.normal(8, 510, rows * 256).reshape(rows, 256).astype(F32) * F32(1.3)
    sel, sc = synth.moe_routes(8, 520, rows, experts, top_k, dtype=F32)
    return x, sel, sc, bank


def test_moe_input_is_read_as_f16():
    """half(x) first: f32 and bf16 inputs give exactly the result of their f16
    rounding (values chosen off the f16 grid, so skipping the cast shows)."""
    x, sel, sc, bank = moe_case()
    sc16 = sc.astype(F16)
    assert not np.array_equal(x.astype(F16).astype(F32), x)
    want = oracle.moe_forward(x.astype(F16), sel, sc16, *bank, 3, 0)
    np.testing.assert_array_equal(oracle.moe_forward(x, sel, sc16, *bank, 3, 0), want)
    xb = bf16_bits(x)
    np.testing.assert_array_equal(
        oracle.moe_forward(xb, sel, sc16, *bank, 3, 0, x_dtype="bf16"),
        oracle.moe_forward(bf16_value(xb).astype(F16), sel, sc16, *bank, 3, 0))


def test_moe_score_promotion_is_exact():
    """Each slot's f16 expert output d_t is read back through one-hot f16 scores
    (score 1 on slot t, 0 elsewhere: the f16 products are exact and the f32 sum
    of one value and zeros is that value).  Then f32 scores must give
    sum_t float32(d_t) * s_t in f32 (t order), bf16 scores the same with
    s_t = float32(bf16(s)), and f16 scores f16(sum_t f32(f16(d_t * s_t)))."""
    x, sel, sc, bank = moe_case()
    rows, top_k = sc.shape
    d = []
    for t in range(top_k):
        onehot = np.zeros((rows, top_k), F16)
        onehot[:, t] = 1
        d.append(oracle.moe_forward(x, sel, onehot, *bank, 3, 0).astype(F32))
    want32 = np.zeros_like(d[0])
    for t in range(top_k):
        want32 = want32 + d[t] * sc[:, t:t + 1]
    got32 = oracle.moe_forward(x, sel, sc, *bank, 3, 0)
    assert got32.dtype == F32
    np.testing.assert_array_equal(got32, want32)
    sb = bf16_bits(sc)
    wantb = np.zeros_like(d[0])
    for t in range(top_k):
        wantb = wantb + d[t] * bf16_value(sb[:, t:t + 1])
    np.testing.assert_array_equal(oracle.moe_forward(x, sel, sb, *bank, 3, 0, scores_dtype="bf16"),
                                  wantb)
    sc16 = sc.astype(F16)
    want16 = np.zeros_like(d[0])
    for t in range(top_k):
        want16 = want16 + (d[t] * sc16[:, t:t + 1].astype(F32)).astype(F16).astype(F32)
    got16 = oracle.moe_forward(x, sel, sc16, *bank, 3, 0)
    assert got16.dtype == F16
    np.testing.assert_array_equal(got16, want16.astype(F16))
    # the f32 result keeps what the f16 products and the f16 result round away
    assert not np.array_equal(got32, got16.astype(F32))


def test_finish_and_reduce_score_dtypes():
    rng = np.random.default_rng(3)
    rows, top_k, width = 3, 2, 256
    raw = rng.normal(0, 40, (rows * top_k, width)).astype(F32)
    svh = rng.uniform(0.5, 1.5, (rows * top_k, width)).astype(F16)
    sc = rng.uniform(0, 1, (rows, top_k)).astype(F32)
    d = []
    for t in range(top_k):
        onehot = np.zeros((rows, top_k), F16)
        onehot[:, t] = 1
        d.append(oracle.finish_and_reduce(raw, svh, onehot).astype(F32))
    want = d[0] * sc[:, :1] + d[1] * sc[:, 1:2]
    np.testing.assert_array_equal(oracle.finish_and_reduce(raw, svh, sc), want)
    sb = bf16_bits(sc)
    wantb = d[0] * bf16_value(sb[:, :1]) + d[1] * bf16_value(sb[:, 1:2])
    np.testing.assert_array_equal(oracle.finish_and_reduce(raw, svh, sb, scores_dtype="bf16"),
                                  wantb)
