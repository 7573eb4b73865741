"""The direct-Metal projection ops of the codec driver, replayed on checkpoints
built the way the reference's physical harnesses build theirs.

* tests/physical_flash_projection.py:16-132 (seed 7503): a qwen4_exp checkpoint
  with one projection per K in 1..8 and codebook (input 128/640/2560/4096, 128
  or 256 columns; F32 / BF16 / F16 scales by codebook; legacy su/sv names for
  K % 3 == 0; U16 trellis for odd K, I16 for even; an F16 bias for odd K), two
  dense experts assembled from those projections (one with a down projection
  of the wrong width) and an 8192 x 128 projection that the direct path's split
  policy refuses; metal-checkpoint-linear on 1 or 3 rows, the reversed and
  padded f16 / f32 views of the codebook-1 inputs, metal-checkpoint-expert on
  1 and 3 rows, metal-exl3-linear on the same projections of the checkpoint
  declared generic (qwen3_5_moe) and on the 8192-wide one; the harness's five
  invalid requests and their messages;
* tests/physical_projection_group.py:38-133 (seed 75103): qwen3_5_moe
  checkpoints of three projections (1024, 128 and 256 columns) per K and
  codebook, two wide dense bundles, a mixed-codebook bundle, a single
  projection, a repeated projection and a negative-stride input view;
  metal-checkpoint-group against mlx-checkpoint-group (grouped flag and every
  output word), and the harness's five invalid requests.

The reference's expected words come from its MLX build, which cannot run here.
Each output is instead compared bit for bit with the library's own API on the
same checkpoint (Exl3Linear.from_checkpoint(...).forward, swiglu) and, within
the linear tolerance, with the oracle on the loader-rounded weights.
"""

from __future__ import annotations

import json

import numpy as np
import pytest

import oracle
from codec_client import run
from mlxl3_amd import synth

pytestmark = pytest.mark.gpu

TOL_REL = 1e-3
TOL_ULP = 2
CHAIN_TOL_REL = 5e-3


def bf16_of_f16(v):
    """MLX astype(bfloat16) of f16 values: round to nearest even."""
    bits = np.asarray(v, np.float16).astype(np.float32).view(np.uint32)
    return ((bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1)))
            >> np.uint32(16)).astype(np.uint16)


def f16_of_bf16(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32).astype(np.float16)


def check(y, ref, label, tol=TOL_REL, ulp=TOL_ULP):
    y = np.asarray(y, np.float64)
    r = np.asarray(ref, np.float64)
    rel = np.linalg.norm(y - r) / np.linalg.norm(r)
    ulps = np.abs(y - r).max() / float(np.spacing(np.float16(np.abs(r).max())))
    print(f"{label}: rel_l2={rel:.3e} max_abs={ulps:.2f} ulp", flush=True)
    assert rel <= tol and (ulp is None or ulps <= ulp), (label, rel, ulps)


def flash_fixture(root):
    """The synthetic checkpoint and cases of physical_flash_projection.py,
    with the f16-rounded weights of every projection for the oracle."""
    rng = np.random.default_rng(7503)
    tensors, storage, weights, cases = {}, {}, {}, []

    def case(prefix, width, batch, expert=False):
        x = rng.normal(0, 0.125, (batch, width)).astype(np.float16)
        cases.append({"op": "metal-checkpoint-expert" if expert else "metal-checkpoint-linear",
                      "path": str(root), "prefix": prefix,
                      "x": x.view(np.uint16).ravel().tolist()})

    for k in range(1, 9):
        for mode in range(3):
            prefix = f"layer_k{k}_cb{mode}"
            width = (128, 640, 2560, 4096)[(k + mode) % 4]
            cols = 128 if mode != 2 else 256
            data = rng.integers(0, 65536, (width // 16, cols // 16, 16 * k), dtype=np.uint16)
            tensors[prefix + ".trellis"] = data if k % 2 else data.view(np.int16)
            legacy = k % 3 == 0
            rounded = []
            for role, size in (("su" if legacy else "suh", width), ("sv" if legacy else "svh", cols)):
                factors = rng.normal(0.8, 0.3, size).astype(np.float32 if mode == 0 else np.float16)
                if mode == 1:
                    bits = bf16_of_f16(factors)
                    tensors[f"{prefix}.{role}"] = ("BF16", bits)
                    rounded.append(f16_of_bf16(bits))
                else:
                    tensors[f"{prefix}.{role}"] = factors
                    rounded.append(factors.astype(np.float16))
            if mode:
                tensors[prefix + (".mul1" if mode == 2 else ".mcg")] = np.array([1], np.int32)
            bias = None
            if k % 2:
                bias = rng.normal(0, 0.17, cols).astype(np.float16)
                tensors[prefix + ".bias"] = bias
            storage[prefix] = {"quant_format": "exl3"}
            weights[prefix] = (data, rounded[0], rounded[1], bias, k, mode)
            case(prefix, width, 1 if k % 2 else 3)
    for expert, down in (("synthetic_expert", "layer_k8_cb0"), ("bad_expert", "layer_k1_cb0")):
        for projection, src in (("gate_proj", "layer_k4_cb0"), ("up_proj", "layer_k3_cb1"),
                                ("down_proj", down)):
            dest = f"{expert}.{projection}"
            storage[dest] = {"quant_format": "exl3"}
            weights[dest] = weights[src]
            for name, val in list(tensors.items()):
                if name.startswith(src + "."):
                    tensors[dest + name[len(src):]] = val
    for batch in (1, 3):
        case("synthetic_expert", 128, batch, expert=True)
    tensors["four.trellis"] = np.zeros((512, 8, 16), dtype=np.uint16)
    tensors["four.suh"] = np.ones(8192, dtype=np.float16)
    tensors["four.svh"] = np.ones(128, dtype=np.float16)
    storage["four"] = {"quant_format": "exl3"}
    weights["four"] = (tensors["four.trellis"], tensors["four.suh"], tensors["four.svh"], None, 1, 0)
    synth.write_checkpoint(root, [tensors], storage, model_type="qwen4_exp", bits=None,
                           index=False)
    # reversed, padded views of the codebook-1 inputs (f16 storage, or f32
    # storage one step above each value, which the cast rounds back)
    views = []
    for c in list(cases):
        if not c["prefix"].endswith("cb1"):
            continue
        x = np.asarray(c["x"], np.uint16).view(np.float16)
        rows = 3 if len(x) % 3 == 0 else 1
        width = len(x) // rows
        backing = np.pad(x.reshape(rows, width)[::-1, ::-1], ((0, 0), (1, 2)), constant_values=7)
        use_f32 = (len(cases) + len(views)) % 2 == 0
        if use_f32:
            backing = np.nextafter(backing.astype(np.float32), np.float32(1.0))
        assert np.array_equal(backing[::-1, -3:0:-1].astype(np.float16).view(np.uint16).ravel(),
                              x.view(np.uint16))
        packet = {**c, "x_layout": {"shape": [rows, width], "strides": [-width - 3, -1],
                                    "offset": backing.size - 3}}
        if use_f32:
            del packet["x"]
            packet["x_f32"] = backing.ravel().tolist()
        else:
            packet["x"] = backing.view(np.uint16).ravel().tolist()
        views.append((packet, c))
    return cases, views, weights


def rows_of(c):
    return np.asarray(c["x"], np.uint16).view(np.float16)


def library_linear(ck, prefix, x):
    import torch

    import mlxl3_amd

    lin = mlxl3_amd.Exl3Linear.from_checkpoint(ck, prefix)
    y = lin.forward(torch.from_numpy(np.ascontiguousarray(x)).cuda())
    torch.cuda.synchronize()
    return y.cpu().numpy()


def library_expert(ck, prefix, x):
    import torch

    import mlxl3_amd

    gate, up, down = (mlxl3_amd.Exl3Linear.from_checkpoint(ck, f"{prefix}.{p}_proj")
                      for p in ("gate", "up", "down"))
    xt = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    y = down.forward(mlxl3_amd.swiglu(gate.forward(xt), up.forward(xt)))
    torch.cuda.synchronize()
    return y.cpu().numpy()


def library_bundle(ck, prefixes, x, grouped):
    """Outputs of the projections on one row through the library's API: one
    Exl3Group when the bundle is grouped, else each Exl3Linear."""
    import torch

    import mlxl3_amd

    lins = [mlxl3_amd.Exl3Linear.from_checkpoint(ck, p) for p in prefixes]
    xt = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    ys = mlxl3_amd.Exl3Group(lins)(xt) if grouped else [lin.forward(xt) for lin in lins]
    torch.cuda.synchronize()
    return [y.cpu().numpy() for y in ys]


def oracle_linear(w, x):
    data, suh, svh, bias, k, cb = w
    return oracle.forward(x, data, suh, svh, k, cb, bias=bias, mode=1)


def test_flash_projection_replay(tmp_path):
    import mlxl3_amd

    root = tmp_path / "synthetic"
    cases, views, weights = flash_fixture(root)
    generic = tmp_path / "generic"
    generic.mkdir()
    for f in root.iterdir():
        (generic / f.name).write_bytes(f.read_bytes())
    (generic / "config.json").write_text(json.dumps({"model_type": "qwen3_5_moe"}))
    exl3_cases = [{**c, "path": str(generic), "op": "metal-exl3-linear"}
                  for c in cases if c["op"] == "metal-checkpoint-linear"]
    four_x = np.random.default_rng(1).normal(0, 0.125, (1, 8192)).astype(np.float16)
    exl3_cases.append({"op": "metal-exl3-linear", "path": str(generic), "prefix": "four",
                       "x": four_x.view(np.uint16).ravel().tolist()})
    invalid = [
        ({**cases[0], "x": []}, "invalid Flash projection batch"),
        ({**cases[0], "prefix": "missing"}, "missing projection trellis"),
        ({**cases[0], "prefix": "four"}, "unsupported projection geometry/split count"),
        ({**cases[0], "x": [1]}, "input is not a complete row"),
        ({**cases[0], "op": "metal-checkpoint-expert", "prefix": "bad_expert"},
         "incompatible Flash expert projection geometry"),
        ({**exl3_cases[0], "op": "metal-checkpoint-linear"}, "requires a Flash reference checkpoint"),
    ]
    stream = [r for r, _ in invalid] + cases + [p for p, _ in views] + exl3_cases
    replies = run(stream, timeout=300)
    for (req, message), reply in zip(invalid, replies):
        assert message in reply.get("error", ""), (req["prefix"], reply)
    replies = replies[len(invalid):]
    ck = mlxl3_amd.Checkpoint(root)
    ckg = mlxl3_amd.Checkpoint(generic)
    n_words = 0
    expected = {}
    for c, reply in zip(cases, replies[:len(cases)]):
        assert "data" in reply, (c["prefix"], reply)
        got = np.asarray(reply["data"], np.uint16)
        prefix = c["prefix"]
        expert = c["op"] == "metal-checkpoint-expert"
        width = 128 if expert else weights[prefix][0].shape[0] * 16
        x = rows_of(c).reshape(-1, width)
        mine = library_expert(ck, prefix, x) if expert else library_linear(ck, prefix, x)
        assert np.array_equal(got, mine.view(np.uint16).ravel()), prefix
        assert np.isfinite(got.view(np.float16)).all() and np.any(got != 0), prefix
        if expert:
            w = {p: weights[f"{prefix}.{p}_proj"] for p in ("gate", "up", "down")}
            act = oracle.swiglu(oracle_linear(w["gate"], x), oracle_linear(w["up"], x))
            ref = oracle_linear(w["down"], act)
            check(got.view(np.float16), ref.ravel(), f"expert {prefix} rows={x.shape[0]}",
                  tol=CHAIN_TOL_REL, ulp=None)
        else:
            check(got.view(np.float16), oracle_linear(weights[prefix], x).ravel(),
                  f"linear {prefix} rows={x.shape[0]}")
        expected[(prefix, c["op"])] = got
        n_words += got.size
    replies = replies[len(cases):]
    for (packet, c), reply in zip(views, replies[:len(views)]):
        assert reply == {"data": expected[(c["prefix"], c["op"])].tolist()}, c["prefix"]
    replies = replies[len(views):]
    for c, reply in zip(exl3_cases, replies):
        assert "data" in reply, (c["prefix"], reply)
        got = np.asarray(reply["data"], np.uint16)
        if c["prefix"] == "four":
            # zero trellis words decode to one constant weight per codebook:
            # the library's own output on the same checkpoint, and finite
            mine = library_linear(ckg, "four", four_x)
            assert np.array_equal(got, mine.view(np.uint16).ravel())
            check(got.view(np.float16), oracle_linear(weights["four"], four_x).ravel(), "exl3 four")
        else:
            assert np.array_equal(got, expected[(c["prefix"], "metal-checkpoint-linear")]), c["prefix"]
    print(f"flash replay: {len(cases)} cases, {len(views)} views, {len(exl3_cases)} generic, "
          f"{n_words} words", flush=True)
    ck.close()
    ckg.close()


def group_fixtures(root):
    """The synthetic checkpoints and cases of physical_projection_group.py."""
    rng = np.random.default_rng(75103)
    cases = []

    def fixture(folder, width, widths, k, mode):
        tensors, storage = {}, {}
        for i, cols in enumerate(widths):
            prefix = f"p{i}"
            words = rng.integers(0, 65536, (width // 16, cols // 16, k * 16), dtype=np.uint16)
            tensors[prefix + ".trellis"] = words if k % 2 else words.view(np.int16)
            for suffix, n in (("suh", width), ("svh", cols), ("bias", cols)):
                if mode == 1:
                    tensors[f"{prefix}.{suffix}"] = (
                        "BF16", np.resize(np.array([0x3F00, 0x3F40, 0xBF00, 0x3F80], np.uint16), n))
                else:
                    tensors[f"{prefix}.{suffix}"] = rng.normal(0.7, 0.1, n).astype(
                        np.float32 if mode == 0 else np.float16)
            if mode:
                tensors[prefix + (".mcg" if mode == 1 else ".mul1")] = np.array([1], np.int32)
            storage[prefix] = {"quant_format": "exl3"}
        synth.write_checkpoint(folder, [tensors], storage, model_type="qwen3_5_moe", bits=None,
                               index=False)
        x = rng.normal(0, 0.1, width).astype(np.float16)
        return {"op": "metal-checkpoint-group", "path": str(folder),
                "prefixes": [f"p{i}" for i in range(len(widths))],
                "x": x.view(np.uint16).tolist()}, tensors

    for k in range(1, 9):
        for mode in range(3):
            width = (128, 2048, 8192)[(k + mode) % 3]
            cases.append(fixture(root / f"k{k}-cb{mode}", width, [1024, 128, 256], k, mode)[0])
    for widths in ([10240, 6144], [17408, 17408]):
        cases.append(fixture(root / f"dense-{sum(widths)}", 5120, widths, 2, 2)[0])
    mixed, tensors = fixture(root / "mixed", 2048, [1024, 128], 2, 0)
    tensors["p1.mul1"] = np.array([1], np.int32)
    synth.write_checkpoint(root / "mixed", [tensors], {"p0": {"quant_format": "exl3"},
                                                       "p1": {"quant_format": "exl3"}},
                           model_type="qwen3_5_moe", bits=None, index=False)
    cases.append(mixed)
    first = cases[0]
    cases.append({**first, "prefixes": ["p0"]})
    cases.append({**first, "prefixes": ["p0", "p0"]})
    logical = np.asarray(first["x"], np.uint16).view(np.float16)
    backing = np.zeros(logical.size * 2 + 3, np.float16)
    backing[1:logical.size * 2 + 1:2] = logical[::-1]
    cases.append({**first, "x": backing.view(np.uint16).tolist(),
                  "x_layout": {"shape": [1, logical.size], "strides": [backing.size, -2],
                               "offset": logical.size * 2 - 1}})
    return cases


def test_projection_group_replay(tmp_path):
    import mlxl3_amd

    cases = group_fixtures(tmp_path)
    packet = cases[0]
    invalid = [
        {**packet, "prefixes": []},
        {**packet, "prefixes": ["missing"]},
        {**packet, "x": []},
        {**packet, "x": packet["x"] + [0]},
        {**packet, "prefixes": ["p0", "missing"]},
    ]
    stock = [{**{k: v for k, v in c.items() if k != "x_layout"}, "op": "mlx-checkpoint-group",
              "x": cases[0]["x"] if "x_layout" in c else c["x"]} for c in cases]
    native = run(invalid + cases + [cases[-1]], timeout=300)
    refs = run(stock, timeout=300)
    assert all(r.get("error") for r in native[:len(invalid)]), native[:len(invalid)]
    assert "invalid grouped input row length" in native[2]["error"]
    assert "invalid grouped input row length" in native[3]["error"]
    native = native[len(invalid):]
    assert native[-1] == native[-2]
    compared = 0
    for c, want, got in zip(cases, refs, native[:-1]):
        assert "data" in want and "data" in got, (c["path"], want, got)
        want, got = want["data"], got["data"]
        assert type(got["grouped"]) is bool and got["grouped"] == want["grouped"], c["path"]
        assert len(got["outputs"]) == len(want["outputs"]) == len(c["prefixes"])
        ck = mlxl3_amd.Checkpoint(c["path"])
        x = np.asarray(cases[0]["x"] if "x_layout" in c else c["x"], np.uint16).view(np.float16)
        mine = library_bundle(ck, c["prefixes"], x[None, :], got["grouped"])
        for prefix, a, b, m in zip(c["prefixes"], got["outputs"], want["outputs"], mine):
            a, b = np.asarray(a, np.uint16), np.asarray(b, np.uint16)
            assert np.array_equal(a, b), (c["path"], prefix)
            assert np.isfinite(a.view(np.float16)).all() and np.any(a != 0)
            assert np.array_equal(a, m.view(np.uint16).ravel()), (c["path"], prefix)
            compared += a.size
        ck.close()
    # grouped exactly when two or more projections share K (not 7) and codebook
    flags = [g["data"]["grouped"] for g in native[:-1]]
    assert flags[:24] == [k != 7 for k in range(1, 9) for _ in range(3)]
    assert flags[24:] == [True, True, False, False, True, True]
    print(f"group replay: {len(cases)} cases, {compared} words", flush=True)
