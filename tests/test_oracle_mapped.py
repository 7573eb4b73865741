"""The oracle's expert_mapped (linear.rs:2817-2852) pinned to the oracle's
linear forward, which the golden vectors and closed forms pin: row r of a
mapped call is exactly (bit for bit: the same products summed in the same
order) the linear forward of row r alone on the bank's tile columns
selected[route] * out/16 + p * stride + t, with the row's own suh and svh;
raw returns that forward's f32 yhat.  Rows whose columns leave the bank are
zero.  A mutant that reads the wrong projection stride, the wrong route of a
row or another row's scales fails these equalities."""

import numpy as np
import pytest

import oracle


def bank_case(seed, k, in_f, out, experts, projections, stride):
    rng = np.random.default_rng(seed)
    ot = out // 16
    tiles = (experts - 1) * ot + (projections - 1) * stride + ot
    bank = rng.integers(0, 1 << 16, (in_f // 16, tiles, 16 * k), dtype=np.uint16)
    return rng, bank, tiles


@pytest.mark.parametrize("k, cb, projections, stride, x_dtype", [
    (2, 0, 1, 0, "f16"),
    (3, 1, 2, 40, "f16"),
    (4, 2, 3, 8, "bf16"),
    (5, 0, 2, 16, "f32"),
])
def test_mapped_rows_are_linear_forwards(k, cb, projections, stride, x_dtype):
    in_f, out, experts = 256, 128, 5
    rng, bank, tiles = bank_case(100 + k, k, in_f, out, experts, projections, stride)
    routes = 4
    rows = routes * projections
    selected = rng.integers(0, experts, routes).astype(np.uint32)
    x16 = rng.normal(0, 1, (rows, in_f)).astype(np.float16)
    if x_dtype == "bf16":
        x = (x16.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        kw = {"x_dtype": "bf16"}
    elif x_dtype == "f32":
        x, kw = rng.normal(0, 1, (rows, in_f)).astype(np.float32), {}
    else:
        x, kw = x16, {}
    suh = (rng.random((rows, in_f)) + 0.5).astype(np.float16)
    svh = (rng.random((rows, out)) + 0.5).astype(np.float16)
    y = oracle.expert_mapped(x, suh, bank, selected, projections, out, stride, k, cb, svh=svh, **kw)
    raw = oracle.expert_mapped(x, suh, bank, selected, projections, out, stride, k, cb, raw=True,
                               **kw)
    ot = out // 16
    for r in range(rows):
        route, p = divmod(r, projections)
        base = int(selected[route]) * ot + p * stride
        w = np.ascontiguousarray(bank[:, base:base + ot, :])
        want, yhat = oracle.forward(x[r:r + 1], w, suh[r], svh[r], k, cb, mode=1,
                                    return_yhat=True, **kw)
        assert np.array_equal(y[r:r + 1].view(np.uint16 if y.dtype != np.float32 else np.uint32),
                              want.view(np.uint16 if want.dtype != np.float32 else np.uint32)), r
        assert np.array_equal(raw[r:r + 1].view(np.uint32), yhat.view(np.uint32)), r


def test_mapped_rows_past_the_bank_are_zero():
    k, in_f, out = 2, 128, 128
    rng, bank, tiles = bank_case(7, k, in_f, out, 3, 1, 0)
    selected = np.array([1, 3, 0], np.uint32)  # expert 3 of a 3-expert bank
    x = rng.normal(0, 1, (3, in_f)).astype(np.float16)
    suh = np.ones((3, in_f), np.float16)
    svh = np.ones((3, out), np.float16)
    y = oracle.expert_mapped(x, suh, bank, selected, 1, out, 0, k, 0, svh=svh)
    raw = oracle.expert_mapped(x, suh, bank, selected, 1, out, 0, k, 0, raw=True)
    assert not y[1].any() and not raw[1].any()
    assert y[0].any() and y[2].any()
