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
  mirror's results and the oracle, bit for bit;
* metal-prepare128 and metal-prepare-view on seeded rows, edge values and
  strided views (the case lists are in the docstrings below), bit for bit
  against the oracle's prologue and the library's prepare128.
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


PREP_SEED = 6221


def prepare128_cases():
    """f16 prepare128 cases (input x scale, one f16 product, then the staged
    H128 of every 128-wide block):

    * the 128 unit rows with unit scales, whose outputs are the normalised
      Sylvester rows;
    * rows in (1, 2, 7, 33) x widths (256, 896, 4096) of N(0, 1) inputs with
      1% outlier channels scaled by 20, with column scales (one row) when
      rows + width / 128 is even, element scales (one per input) when it is
      odd, and both for 7 rows; scales +-U(0.5, 1.5);
    * edge rows: all negative zeros, the smallest subnormals between signed
      zeros, the largest subnormal beside the smallest normal, and signed
      ones mixed with subnormals, under unit scales and, by element, under
      scales of -1 and 2**-10 (which push the products into the subnormals).
    """
    cases = [("unit-rows", np.eye(128, dtype=np.float16), np.ones((1, 128), dtype=np.float16))]
    tid = 0
    for rows in (1, 2, 7, 33):
        for width in (256, 896, 4096):
            x = synth.activations(PREP_SEED, tid, rows, width, outlier_frac=0.01)
            kinds = (1, rows) if rows == 7 else ((1,) if (rows + width // 128) % 2 == 0 else (rows,))
            for scale_rows in kinds:
                s = synth.signs_scales(PREP_SEED, tid + 1 + scale_rows, scale_rows * width)
                cases.append((f"normal-{rows}x{width}-scales-{scale_rows}", x,
                              s.reshape(scale_rows, width)))
            tid += 64
    edge = np.zeros((4, 256), np.uint16)
    edge[0] = 0x8000
    edge[1, 0::4], edge[1, 1::4], edge[1, 2::4], edge[1, 3::4] = 0x0001, 0x8000, 0x8001, 0x0000
    edge[2, 0::2], edge[2, 1::2] = 0x03FF, 0x8400
    edge[3] = np.resize(np.array([0x3C00, 0x8002, 0xBC00, 0x0200, 0x83FF], np.uint16), 256)
    x = edge.view(np.float16)
    cases.append(("edge-unit-scales", x, np.ones((1, 256), np.float16)))
    flip = np.resize(np.array([-1.0, 2.0 ** -10, 1.0], np.float16), (4, 256))
    cases.append(("edge-element-scales", x, np.ascontiguousarray(flip)))
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


def off_by_a_little(v16):
    """float32 values one f32 step away from each non-zero f16 value (away from
    zero), which a round-to-nearest cast takes back to the f16 value; zeros
    keep their sign."""
    v = np.asarray(v16, np.float16).astype(np.float32)
    return np.where(v == 0, v, np.nextafter(v, np.copysign(np.float32(np.inf), v)))


def view_layout(view, backing):
    """Element shape, strides and offset of a numpy view into `backing`."""
    item = backing.itemsize
    return {"shape": list(view.shape), "strides": [b // item for b in view.strides],
            "offset": (view.__array_interface__["data"][0]
                       - backing.__array_interface__["data"][0]) // item}


def test_prepare_view_strided_views_match_the_oracle():
    """metal-prepare-view on views of f16 and f32 storage (the f32 values one
    f32 step off f16 values, so the cast rounds them back): widths (256, 1152,
    3072) with 2, 3 and 5 rows, each input view paired with a scale view of
    the same shape:

    * column-major input (a transposed backing) with element scales read
      backwards along each row;
    * rows taken bottom-up from every second backing row, columns right to
      left, with column-major scales;
    * one backing row repeated for every row (row stride 0) with scales of
      one row repeated the same way;
    * one backing column repeated along the row (column stride 0) with every
      other element of a scale row.

    Every backing has guard elements around the viewed region; the outputs are
    compared bit for bit with the oracle on the gathered rows.
    """
    reqs, wants, names = [], [], []
    tid = 0
    for width, rows in ((256, 2), (1152, 3), (3072, 5)):
        for dtype in (np.float16, np.float32):
            base16 = (synth.normal(PREP_SEED, 500 + tid, (2 * rows + 3) * (width + 4)) * 0.75
                      ).astype(np.float16).reshape(2 * rows + 3, width + 4)
            tall16 = (synth.normal(PREP_SEED, 600 + tid, (width + 4) * (rows + 3))
                      .astype(np.float16).reshape(width + 4, rows + 3))
            scales = synth.signs_scales(PREP_SEED, 700 + tid, (2 * width + 5) * (rows + 2)).reshape(
                rows + 2, 2 * width + 5)
            tscales = np.ascontiguousarray(scales[:, :width + 3].T)  # [width + 3, rows + 2]
            tid += 1
            for kind in range(4):
                if kind == 0:
                    backing, x = tall16, tall16[2:2 + width, 1:1 + rows].T
                    sb, sv = scales, scales[1:1 + rows, width + 1:1:-1]
                elif kind == 1:
                    backing, x = base16, base16[2 * rows - 1:0:-2, width + 2:2:-1]
                    sb, sv = tscales, tscales[2:2 + width, 1:1 + rows].T
                elif kind == 2:
                    backing = base16
                    x = np.broadcast_to(base16[rows, 3:3 + width], (rows, width))
                    sb, sv = scales, np.broadcast_to(scales[rows, 4:4 + width], (rows, width))
                else:
                    backing = tall16
                    x = np.broadcast_to(tall16[1:1 + rows, 2, None], (rows, width))
                    sb, sv = scales, np.broadcast_to(scales[0, 3:3 + 2 * width:2], (rows, width))
                assert x.shape == sv.shape == (rows, width)
                layout = view_layout(x, backing)
                if dtype == np.float32:
                    store = off_by_a_little(backing).ravel()
                    idx = (layout["offset"] + np.arange(rows)[:, None] * layout["strides"][0]
                           + np.arange(width)[None, :] * layout["strides"][1])
                    assert np.array_equal(store[idx].astype(np.float16).view(np.uint16),
                                          np.ascontiguousarray(x).view(np.uint16))
                    field, raw = "x_f32", store.tolist()
                else:
                    field, raw = "x", backing.view(np.uint16).ravel().tolist()
                reqs.append({"op": "metal-prepare-view", field: raw, "x_layout": layout,
                             "scale_layout": view_layout(sv, sb),
                             "data": sb.view(np.uint16).ravel().tolist()})
                xs = np.ascontiguousarray(x)
                ss = np.ascontiguousarray(sv)
                wants.append(np.concatenate([oracle.prologue(xs[r:r + 1], ss[r])
                                             for r in range(rows)]))
                names.append(f"kind{kind}-{rows}x{width}-{np.dtype(dtype).name}")
    rows_out = run(reqs)
    for name, want, row in zip(names, wants, rows_out):
        got = np.array(row["data"], np.uint16)
        bad = int((got != want.view(np.uint16).ravel()).sum())
        print(f"prepare-view {name}: {bad} of {got.size} differ", flush=True)
        assert bad == 0, name
