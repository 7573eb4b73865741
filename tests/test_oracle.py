"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each check is independent of the oracle's own code: the reference's golden
vectors (tests/golden/, see make_golden.py), closed forms evaluated by numpy,
library routines (numpy's IEEE float16, torch's bfloat16), brute force on small
inputs, and invariants the format fixes.
"""

import json

import numpy as np
import pytest

import oracle


def f16(bits):
    return np.asarray(bits, np.uint16).view(np.float16)


# ---------------------------------------------------------------------------
# scalar conversions against numpy / torch
# ---------------------------------------------------------------------------


def test_f16_to_f32_exhaustive_matches_numpy():
    L = oracle.lib()
    bits = np.arange(65536, dtype=np.uint16)
    ours = np.array([L.exl3o_f16_to_f32(int(b)) for b in bits], np.float32)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rounding_matches_numpy():
    L = oracle.lib()
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
        # every f16 value, its neighbours and the exact midpoints (ties)
        np.arange(0, 0x7C00, 7, dtype=np.uint16).view(np.float16).astype(np.float32),
        ((np.arange(0, 0x7BFF, 13, dtype=np.uint16).view(np.float16).astype(np.float64)
          + np.arange(1, 0x7C00, 13, dtype=np.uint16).view(np.float16).astype(np.float64)) / 2
         ).astype(np.float32),
        np.float32([65504, 65519.99, 65520, 1e9, 6e-8, 2.98e-8, 5.96e-8, 0.0, -0.0, np.inf, -np.inf]),
    ])
    vals = np.concatenate([vals, -vals]).astype(np.float32)
    ours = np.array([L.exl3o_f32_to_f16(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    L = oracle.lib()
    rng = np.random.default_rng(2)
    vals = (rng.standard_normal(20000) * 10.0 ** rng.integers(-20, 20, 20000)).astype(np.float32)
    ours = np.array([L.exl3o_f32_to_bf16(float(v)) for v in vals], np.uint16)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


# ---------------------------------------------------------------------------
# codebooks
# ---------------------------------------------------------------------------


def numpy_codebook(cb):
    """Closed form of codec.rs:52-71 evaluated with numpy's float16 arithmetic."""
    x = np.arange(65536, dtype=np.uint64)
    if cb == 2:
        p = (x * np.uint64(0x83DCD12D)) & np.uint64(0xFFFFFFFF)
        s = 0x6400 + sum(((p >> np.uint64(8 * i)) & np.uint64(255)) for i in range(4))
        h = s.astype(np.uint16).view(np.float16).astype(np.float64)
        inv = np.uint16(0x1EEE).view(np.float16).astype(np.float64)
        bias = np.uint16(0xC931).view(np.float16).astype(np.float64)
        return (h * inv + bias).astype(np.float16)  # exact in f64, one rounding
    mult = 89226354 if cb == 0 else 0xCBAC1FED
    add = 64248484 if cb == 0 else 0
    y = (x * np.uint64(mult) + np.uint64(add)) & np.uint64(0xFFFFFFFF)
    z = np.uint64(0x3B603B60) ^ (y & np.uint64(0x8FFF8FFF))
    lo = (z & np.uint64(0xFFFF)).astype(np.uint16).view(np.float16)
    hi = (z >> np.uint64(16)).astype(np.uint16).view(np.float16)
    return lo + hi  # numpy float16 addition: one correct rounding


@pytest.mark.parametrize("cb", [0, 1, 2])
def test_codebook_exhaustive_matches_numpy_closed_form(cb):
    ours = oracle.codebook(cb)
    ref = numpy_codebook(cb).view(np.uint16)
    assert np.array_equal(ours, ref)
    assert np.isfinite(ours.view(np.float16)).all()  # codec.rs:274-281


def test_mul1_matches_reference_table(golden):
    """ar33_codeword_table.metal: RNE f16 of ((1024+i)*887 - 1329*1024)/131072."""
    table = json.loads((golden / "tables.json").read_text())["mul1_sum_to_f16"]
    cb = oracle.codebook(2)
    x = np.arange(65536, dtype=np.uint64)
    p = (x * np.uint64(0x83DCD12D)) & np.uint64(0xFFFFFFFF)
    s = sum(((p >> np.uint64(8 * i)) & np.uint64(255)) for i in range(4)).astype(np.int64)
    assert np.array_equal(cb, np.asarray(table, np.uint16)[s])
    # and the rational closed form, independently
    exact = ((1024 + np.arange(1021)) * 887 - 1329 * 1024) / 131072.0
    assert np.array_equal(exact.astype(np.float16).view(np.uint16), np.asarray(table, np.uint16))


def test_3inst_halves_add_is_exact_in_f32():
    """Both addends lie in [2^-3, 2): the f32 sum is exact, one f16 rounding suffices."""
    x = np.arange(65536, dtype=np.uint64)
    y = (x * np.uint64(89226354) + np.uint64(64248484)) & np.uint64(0xFFFFFFFF)
    z = np.uint64(0x3B603B60) ^ (y & np.uint64(0x8FFF8FFF))
    lo = (z & np.uint64(0xFFFF)).astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (z >> np.uint64(16)).astype(np.uint16).view(np.float16).astype(np.float64)
    assert np.all((np.abs(lo) >= 0.125) & (np.abs(lo) < 2) & (np.abs(hi) >= 0.125) & (np.abs(hi) < 2))
    s32 = lo.astype(np.float32) + hi.astype(np.float32)
    assert np.array_equal(s32.astype(np.float64), lo + hi)


# ---------------------------------------------------------------------------
# golden vectors: quantizer corpus and real checkpoint tiles
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("k", range(2, 9))
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_quantizer_corpus(golden, k, cb):
    d = golden / "quantizer"
    packed = np.fromfile(d / f"oracle-{k}-{cb}-packed.u16", "<u2")
    states = np.fromfile(d / f"oracle-{k}-{cb}-states.u16", "<u2").reshape(-1, 256)
    decoded = np.fromfile(d / f"oracle-{k}-{cb}-decoded.f32", "<f4").reshape(-1, 256)
    assert packed.size == 4 * 16 * k and states.shape == (4, 256)
    assert np.array_equal(oracle.unpack(packed, k), states)
    assert np.array_equal(oracle.pack(states, k).ravel(), packed)
    table = oracle.codebook(cb)
    vals = table[states].view(np.float16).astype(np.float32)
    assert np.array_equal(vals.view(np.uint32), decoded.view(np.uint32))


@pytest.mark.parametrize("name", ["flash", "qwen-dense", "qwen-moe", "lfm-moe"])
def test_real_checkpoint_tiles(golden, name):
    """native/tests/contracts.rs:617-669 over the frozen real tiles."""
    fix = json.loads((golden / "real_tiles" / f"{name}.json").read_text())
    k, cb = fix["k"], fix["mode"]
    table = oracle.codebook(cb)
    perm = oracle.permutation()
    for tile in fix["tiles"]:
        packed = np.asarray(tile["packed"], np.uint16)
        states = oracle.unpack(packed, k)[0]
        assert np.array_equal(states, np.asarray(tile["states"], np.uint16))
        assert np.array_equal(table[states], np.asarray(tile["f16_bits"], np.uint16))
        # basis rows: the tile reconstructed to row-major equals the permuted values
        w = oracle.reconstruct_inner(packed, k, cb, 16, 16)
        expect = np.empty(256, np.uint16)
        expect[perm] = np.asarray(tile["f16_bits"], np.uint16)
        assert np.array_equal(w.view(np.uint16).ravel(), expect)


# ---------------------------------------------------------------------------
# codec invariants (codec.rs:192-248)
# ---------------------------------------------------------------------------


def brute_unpack(packed, k):
    """Definition: 16-bit window ending at bit (t+1)k of the circular stream."""
    bits = []
    p = np.asarray(packed, np.uint16)
    for i in range(8 * k):
        word = int(p[2 * i]) | (int(p[2 * i + 1]) << 16)
        bits += [(word >> (31 - b)) & 1 for b in range(32)]
    total = 256 * k
    out = []
    for t in range(256):
        end = (t + 1) * k
        v = 0
        for b in range(end - 16, end):
            v = (v << 1) | bits[b % total]
        out.append(v)
    return np.asarray(out, np.uint16)


@pytest.mark.parametrize("k", range(1, 9))
def test_unpack_matches_bitstream_definition(k):
    rng = np.random.default_rng(k)
    packed = rng.integers(0, 65536, 16 * k, dtype=np.uint16)
    assert np.array_equal(oracle.unpack(packed, k)[0], brute_unpack(packed, k))


def test_pack_tail_biting_all_bitrates():
    """codec.rs:196-211."""
    src = ((np.arange(768) * 391 + 1729) & 0xFFFF).astype(np.uint16)
    for k in range(1, 9):
        packed = oracle.pack(src, k)
        dec = oracle.unpack(packed, k).ravel()
        mask = (1 << k) - 1
        assert np.array_equal(dec & mask, src & mask)
        assert np.array_equal(oracle.pack(dec, k), packed)
    with pytest.raises(ValueError):
        oracle.pack(src, 0)
    with pytest.raises(ValueError):
        oracle.pack(src[:255], 4)
    with pytest.raises(ValueError):
        oracle.unpack(np.zeros(15, np.uint16), 1)


def test_permutation_bijective_and_reference_positions(golden):
    perm = oracle.permutation()
    assert sorted(perm.tolist()) == list(range(256))
    positions = json.loads((golden / "tables.json").read_text())["reference_positions"]
    assert perm.tolist() == positions
    for row in range(16):  # codec.rs:238-244 lane formula
        for col in range(16):
            lane = (row % 8) // 2 + (col % 8) * 4
            index = lane * 8 + (col // 8) * 4 + (row // 8) * 2 + row % 2
            assert perm[index] == row * 16 + col


# ---------------------------------------------------------------------------
# Hadamard-128
# ---------------------------------------------------------------------------


def sylvester():
    i = np.arange(128)
    return np.where(np.bitwise_count(i[:, None] & i[None, :]) % 2, -1.0, 1.0)


@pytest.mark.parametrize("case", ["matrix-0", "matrix-1", "matrix-4", "activations"])
def test_h128_f32_bit_exact_vs_mlx_fixture(golden, case):
    d = np.load(golden / "hadamard" / "hadamard.npz", allow_pickle=False)
    x = d[f"{case}-input"]
    if case == "activations":
        x = x * d["activations-su"]
    ours = oracle.h128_f32(x.reshape(-1, 128)).reshape(x.shape)
    assert np.array_equal(ours.view(np.uint32), d[f"{case}-output"].view(np.uint32))


def test_h128_staged_is_the_transform_within_f16_rounding():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((64, 128)).astype(np.float16).astype(np.float32)
    ours = oracle.h128_staged(x)
    exact = x.astype(np.float64) @ sylvester() / np.sqrt(128)
    # two interior f16 roundings + the final one: a few f16 ulps of |exact| max
    assert np.abs(ours - exact).max() <= 4 * np.spacing(np.float16(np.abs(exact).max()))
    assert np.array_equal(ours, ours.astype(np.float16).astype(np.float32))


def test_h128_staged_rounding_schedule():
    """Interior roundings sit after strides 8 and 64: f16 rounding of the two
    partial transforms (H16 on contiguous 16-blocks, then H8 across them)."""
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((32, 128)) * 3).astype(np.float16).astype(np.float64)
    i16 = np.arange(16)
    h16 = np.where(np.bitwise_count(i16[:, None] & i16[None, :]) % 2, -1.0, 1.0)
    i8 = np.arange(8)
    h8 = np.where(np.bitwise_count(i8[:, None] & i8[None, :]) % 2, -1.0, 1.0)
    a = (x.reshape(32, 8, 16) @ h16).astype(np.float16).astype(np.float64)  # exact then 1 rounding
    b = np.einsum("rjc,jk->rkc", a, h8).astype(np.float16).astype(np.float64)
    s = np.float32(1 / np.sqrt(128))
    ref = (b.reshape(32, 128).astype(np.float32) * s).astype(np.float16).astype(np.float32)
    assert np.array_equal(oracle.h128_staged(x.astype(np.float32)), ref)


# ---------------------------------------------------------------------------
# forward
# ---------------------------------------------------------------------------


def small_layer(seed, n_in, n_out, k):
    rng = np.random.default_rng(seed)
    tr = rng.integers(0, 65536, (n_in // 16, n_out // 16, 16 * k), dtype=np.uint16)
    suh = (rng.choice([-1, 1], n_in) * rng.uniform(0.5, 1.5, n_in)).astype(np.float16)
    svh = (rng.choice([-1, 1], n_out) * rng.uniform(0.5, 1.5, n_out)).astype(np.float16)
    return tr, suh, svh


@pytest.mark.parametrize("k,cb", [(4, 0), (3, 1), (2, 2), (8, 0)])
def test_forward_mode0_matches_dense_numpy_path(k, cb):
    """ref/forward.py:14-49 restated with a dense W and matrix Hadamards.

    The inner product is checked against f64 separately; the f16 stages are
    then checked exactly given the oracle's own f32 inner product."""
    tr, suh, svh = small_layer(5, 256, 384, k)
    x = np.random.default_rng(6).standard_normal((3, 256)).astype(np.float16)
    W = oracle.reconstruct_inner(tr, k, cb, 256, 384).astype(np.float64)
    H32 = (sylvester() * np.float32(1 / np.sqrt(128))).astype(np.float64)
    xs = x.astype(np.float64) * suh.astype(np.float64)
    xh = np.concatenate([xs[:, b:b + 128] @ H32 for b in range(0, 256, 128)], 1).astype(np.float16)
    ours, yhat = oracle.forward(x, tr, suh, svh, k, cb, mode=0, return_yhat=True)
    exact = xh.astype(np.float64) @ W
    assert np.abs(yhat - exact).max() <= 1e-6 * np.abs(exact).max()
    y = yhat.astype(np.float16).astype(np.float64)
    out = np.concatenate([y[:, b:b + 128] @ H32 for b in range(0, 384, 128)], 1)
    out = (out * svh.astype(np.float64)).astype(np.float16)
    # the oracle rounds f64 -> f32 -> f16 at the end: at most 1 ulp apart
    diff = np.abs(ours.astype(np.float64) - out.astype(np.float64))
    assert (diff <= np.spacing(np.abs(out)).astype(np.float64)).all()
    assert (diff == 0).mean() > 0.99


def test_forward_yhat_is_xhat_times_dense_w():
    k, cb = 4, 0
    tr, suh, svh = small_layer(7, 512, 256, k)
    x = np.random.default_rng(8).standard_normal((2, 512)).astype(np.float16)
    _, yhat = oracle.forward(x, tr, suh, svh, k, cb, mode=1, return_yhat=True)
    xh = oracle.prologue(x, suh).astype(np.float64)
    W = oracle.reconstruct_inner(tr, k, cb, 512, 256).astype(np.float64)
    ref = xh @ W
    assert np.abs(yhat - ref).max() <= 1e-5 * np.abs(ref).max()


def test_forward_modes_agree_within_stated_tolerance():
    k, cb = 4, 0
    tr, suh, svh = small_layer(9, 1024, 512, k)
    x = np.random.default_rng(10).standard_normal((4, 1024)).astype(np.float16)
    y0 = oracle.forward(x, tr, suh, svh, k, cb, mode=0).astype(np.float64)
    y1 = oracle.forward(x, tr, suh, svh, k, cb, mode=1).astype(np.float64)
    rel = np.linalg.norm(y1 - y0) / np.linalg.norm(y0)
    assert rel < 2e-3, rel


def test_forward_dtypes_and_bias():
    k, cb = 4, 0
    tr, suh, svh = small_layer(11, 256, 256, k)
    bias = np.random.default_rng(12).standard_normal(256).astype(np.float16)
    x16 = np.random.default_rng(13).standard_normal((2, 256)).astype(np.float16)
    y16 = oracle.forward(x16, tr, suh, svh, k, cb, bias=bias)
    y16nb = oracle.forward(x16, tr, suh, svh, k, cb)
    ref = (y16nb.astype(np.float32) + bias.astype(np.float32)).astype(np.float16)
    assert np.array_equal(y16.view(np.uint16), ref.view(np.uint16))
    y32 = oracle.forward(x16.astype(np.float32), tr, suh, svh, k, cb)
    assert np.array_equal(y32.astype(np.float16).view(np.uint16), y16nb.view(np.uint16))


def test_forward_rejects_bad_arguments():
    tr, suh, svh = small_layer(14, 128, 128, 4)
    with pytest.raises(ValueError):
        oracle.forward(np.zeros((1, 128), np.float16), tr, suh, svh, 9, 0)
    with pytest.raises(ValueError):
        oracle.forward(np.zeros((1, 128), np.float16), tr, suh, svh, 4, 3)
