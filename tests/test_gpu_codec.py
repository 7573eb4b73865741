"""The codec JSON-lines driver's GPU operations (codec_loop, native/src/main.rs).

* The replay of the reference's check-metal-tiles harness
  (docs/native-coverage/baselines/exl3/check-metal-tiles.py.txt), built the same
  way from the same frozen real tiles: a first request with K = 0 that must
  answer {"error": "K must be in 1..=8, got 0"}, then per tile one
  metal-decode (states and f16 values equal to the fixture) and 16 one-hot
  metal-qmv rows (row i of the tile's row-major matrix, exact: one product
  per output), 205 lines in all;
* unpack / codebook against the oracle on the reference's quantizer vectors and
  on every state; mlx-linear / mlx-group / metal-swiglu against the Python
  mirror's results and the oracle, bit for bit.
"""

import json

import numpy as np
import pytest

import oracle
from codec_client import run
from mlxl3_amd import synth

pytestmark = pytest.mark.gpu


def row_major(bits):
    """kernel_order_to_row_major: stored index i sits at permutation()[i]."""
    m = np.zeros(256, np.uint16)
    m[oracle.permutation()] = np.asarray(bits, np.uint16)
    return m.reshape(16, 16)


def test_check_metal_tiles_replay(golden):
    requests = [{"op": "metal-decode", "k": 0, "data": []}]
    expected = []
    for name in ("flash", "qwen-dense", "qwen-moe", "lfm-moe"):
        fix = json.loads((golden / "real_tiles" / f"{name}.json").read_text())
        assert len(fix["tiles"]) == 3
        for tile in fix["tiles"]:
            args = dict(data=tile["packed"], k=fix["k"], mode=fix["mode"])
            requests.append(dict(op="metal-decode", **args))
            expected.append(dict(states=tile["states"], values=tile["f16_bits"]))
            matrix = row_major(tile["f16_bits"])
            assert np.isfinite(matrix.view(np.float16)).all()
            for i in range(16):
                x = [0] * 16
                x[i] = 0x3C00
                requests.append(dict(op="metal-qmv", x=x, cols=16, **args))
                expected.append(matrix[i].tolist())
    rows = run(requests)
    assert len(rows) == len(requests) == 205
    assert rows[0] == {"error": "K must be in 1..=8, got 0"}
    for actual, want in zip(rows[1:], expected):
        assert actual == {"data": want}


def test_unpack_and_codebook(golden):
    sums = json.loads((golden / "quantizer" / "checksums.json").read_text())
    reqs, want = [], []
    for name in sorted(sums):
        if not name.endswith("-packed.u16"):
            continue
        _, k, cb, _ = name.split("-")
        packed = np.fromfile(golden / "quantizer" / name, dtype="<u2")
        states = np.fromfile(golden / "quantizer" / name.replace("packed", "states"), dtype="<u2")
        reqs.append({"op": "unpack", "k": int(k), "mode": int(cb), "data": packed.tolist()})
        want.append(states.tolist())
    every = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    for cb in range(3):
        reqs.append({"op": "codebook", "mode": cb, "data": every.tolist()})
        want.append(oracle.codebook(cb).tolist())
    for row, w in zip(run(reqs), want):
        assert row == {"data": w}


def test_metal_qmv_general_input():
    """Several tiles and a dense x: f32 accumulation in another order than the
    oracle's, so compare within 1 f16 ulp of the largest output."""
    rng = np.random.default_rng(5)
    rows, cols, k, cb = 64, 48, 3, 1
    packed = rng.integers(0, 1 << 16, size=rows // 16 * cols // 16 * 16 * k, dtype=np.uint16)
    x = (rng.standard_normal(rows) * 0.5).astype(np.float16)
    (row,) = run([{"op": "metal-qmv", "k": k, "mode": cb, "cols": cols, "x": x.view(np.uint16).tolist(),
                   "data": packed.tolist()}])
    got = np.array(row["data"], np.uint16).view(np.float16).astype(np.float64)
    w = oracle.reconstruct_inner(packed, k, cb, rows, cols).astype(np.float64)
    ref = x.astype(np.float64) @ w
    assert np.abs(got - ref).max() <= float(np.spacing(np.float16(np.abs(ref).max())))


def test_linear_group_swiglu_ops():
    import torch

    import mlxl3_amd

    n_in, k, cb, m = 256, 2, 0, 3
    tr, suh, svh, _ = synth.linear_layer(4, 1, n_in, 384, k)
    tr2, suh2, svh2, _ = synth.linear_layer(4, 2, n_in, 128, k)
    x = synth.activations(4, 3, m, n_in)
    bits = lambda a: np.ascontiguousarray(a).view(np.uint16).ravel().tolist()  # noqa: E731
    g = synth.activations(5, 1, 1, 1000).ravel()
    u = synth.activations(5, 2, 1, 1000).ravel()
    rows = run([
        {"op": "mlx-linear", "k": k, "mode": cb, "cols": 384, "data": bits(tr), "suh": bits(suh),
         "svh": bits(svh), "x": bits(x)},
        {"op": "mlx-group", "k": k, "mode": cb, "widths": [384, 128], "data": bits(tr) + bits(tr2),
         "suh": bits(suh) + bits(suh2), "svh": bits(svh) + bits(svh2), "x": bits(x)},
        {"op": "metal-swiglu", "x": bits(g), "data": bits(u)},
    ])
    dev = lambda a: torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).cuda()  # noqa: E731
    lin = mlxl3_amd.Exl3Linear(dev(tr), dev(suh), dev(svh), None, k, cb)
    lin2 = mlxl3_amd.Exl3Linear(dev(tr2), dev(suh2), dev(svh2), None, k, cb)
    y = lin.forward(dev(x)).cpu().numpy()
    y2 = lin2.forward(dev(x)).cpu().numpy()
    assert rows[0] == {"data": bits(y)}
    assert rows[1] == {"data": [bits(y), bits(y2)]}
    assert rows[2] == {"data": bits(oracle.swiglu(g, u))}


def prepare128_cases():
    """The cases of the reference's tests/physical_prepare128.py (its f16 ones):
    the 128 basis rows with unit scales, normal rows of widths 128/640/2560 with
    column or element scales, and subnormal / signed-zero rows."""
    rng = np.random.default_rng(75)
    cases = [("all-128-basis-rows", np.eye(128, dtype=np.float16),
              np.ones((1, 128), dtype=np.float16))]
    for rows in (1, 3, 20):
        for width in (128, 640, 2560):
            x = rng.normal(0, 1.125, (rows, width)).astype(np.float16)
            for scale_rows in sorted({1, rows}):
                s = rng.normal(0, 0.75, (scale_rows, width)).astype(np.float16)
                cases.append((f"mixed-{rows}x{width}-scale-rows-{scale_rows}", x, s))
    bits = np.array([0x0000, 0x8000, 1, 0x8001, 0x3C00, 0xBC00, 0x0400, 0x8400], dtype=np.uint16)
    special = np.resize(bits, (3, 128)).view(np.float16)
    special[1] = np.float16(-0.0)
    special[2] = np.resize(bits[::-1], 128).view(np.float16)
    cases.append(("subnormal-signed-zero", special, np.ones_like(special)))
    return cases


def prepare128_oracle(x, s):
    if s.shape[0] == 1:
        return oracle.prologue(x, s[0])
    return np.concatenate([oracle.prologue(x[r:r + 1], s[r]) for r in range(x.shape[0])])


def test_prepare128_codec_and_abi_match_the_oracle():
    import torch

    import mlxl3_amd

    cases = prepare128_cases()
    reqs = [{"op": "metal-prepare128", "cols": int(x.shape[1]),
             "x": x.view(np.uint16).ravel().tolist(), "data": s.view(np.uint16).ravel().tolist()}
            for _, x, s in cases]
    rows = run(reqs)
    for (name, x, s), row in zip(cases, rows):
        want = np.asarray(prepare128_oracle(x, s)).view(np.uint16).ravel()
        got = np.array(row["data"], dtype=np.uint16)
        bad = np.flatnonzero(got != want)
        print(f"prepare128 {name}: {bad.size} of {want.size} differ", flush=True)
        assert bad.size == 0, (name, bad[:5])
        out = mlxl3_amd.prepare128(torch.from_numpy(x).cuda(),
                                   torch.from_numpy(np.ascontiguousarray(s if s.shape[0] > 1 else s[0])).cuda())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy().view(np.uint16).ravel(), want)
    # basis rows: xhat is the normalised Sylvester row (exact in f16)
    basis = np.asarray(prepare128_oracle(*cases[0][1:])).astype(np.float64)
    assert np.all(np.abs(np.abs(basis) - 2 ** -3.5) < 2 ** -14)


def test_prepare_view_strided_views_match_the_oracle():
    """The view cases of the reference's physical_prepare128.py: transposed,
    reversed, negative-stride and broadcast views of f16 and f32 storage with
    guard words around each backing array, against the oracle on the gathered
    rows (element scales)."""
    rng = np.random.default_rng(75)
    reqs, wants, names = [], [], []
    for width in (128, 640, 2560):
        rows = 3
        for dtype in (np.float16, np.float32):
            base = rng.normal(0, 0.5, (2 * width + 2, rows + 2)).astype(dtype)
            scales = rng.normal(0, 0.75, (rows + 2, width + 2)).astype(np.float16)
            for name, x, sv in (
                ("transpose-reverse", base[1:-1:2, -2:0:-1].T, scales[1:-1, -2:0:-1]),
                ("negative-row-col", base[-2:0:-2, -2:0:-1].T, scales[-2:0:-1, 1:-1]),
                ("row-broadcast", np.broadcast_to(base[1:-1:2, 1], (rows, width)), scales[1:-1, 1:-1]),
                ("column-broadcast", np.broadcast_to(base[1, 1:-1, None], (rows, width)),
                 np.broadcast_to(scales[1, 1:-1], (rows, width))),
            ):
                def layout(view, backing):
                    return {"shape": list(view.shape),
                            "strides": [v // view.itemsize for v in view.strides],
                            "offset": (view.ctypes.data - backing.ctypes.data) // view.itemsize}

                field = "x" if dtype == np.float16 else "x_f32"
                raw = base.view(np.uint16) if dtype == np.float16 else base
                reqs.append({"op": "metal-prepare-view", field: raw.ravel().tolist(),
                             "x_layout": layout(x, base), "scale_layout": layout(sv, scales),
                             "data": scales.view(np.uint16).ravel().tolist()})
                xs = np.ascontiguousarray(x).astype(np.float16)
                ss = np.ascontiguousarray(sv)
                wants.append(np.concatenate([oracle.prologue(xs[r:r + 1], ss[r]) for r in range(rows)]))
                names.append(f"{name}-{width}-{dtype.__name__}")
    rows_out = run(reqs)
    for name, want, row in zip(names, wants, rows_out):
        got = np.array(row["data"], np.uint16)
        bad = int((got != want.view(np.uint16).ravel()).sum())
        print(f"prepare-view {name}: {bad} of {got.size} differ", flush=True)
        assert bad == 0, name
