"""The direct projection ops of the codec driver (metal-checkpoint-linear,
metal-checkpoint-expert, metal-exl3-linear, metal-checkpoint-group) on seeded
synthetic checkpoints.  The ops are those of the reference's codec
(main.rs:1173-1199, :1304-1337); the geometry checks are its direct path's
(gpu/projection.rs:134-333, :2386-2443).

Case matrix of the projection checkpoint (model_type qwen4_exp, seed SEED),
one projection per K in 1..8 and codebook cb in 0..2, i = 3 (K - 1) + cb:

  input width       WIDTHS[i % 5]                 256, 1152, 3072, 640, 5120
  output columns    128 (1 + K % 3)               128, 256, 384
  scale storage     SCALES[(K + cb) % 3]          F16, BF16, F32 (F32 values a
                                                  fraction of an f16 ulp off,
                                                  so the loader's rounding is
                                                  exercised)
  scale names       legacy su / sv when i % 4 == 2, suh / svh otherwise
  trellis dtype     I16 when i is even, U16 when odd
  bias (F16)        when (i // 2) is even
  rows              1 + 5 i % 4 (1..4); 33 rows for i in (5, 14), the
                    multi-row kernel's side of the dispatch
  input             N(0, 1/8) rows; for i % 6 == 5 the first row also
                    carries f16 subnormals and the last row negative zeros

plus two dense experts of input 512 / hidden 768 (gate K3 MCG BF16, up K5
3INST F32 legacy names, down K2 MUL1 F16 with bias; "mlp.bad" has a 384-wide
down projection) on 1 and 3 rows, and "wide", 12288 x 256, which the direct
path's split policy refuses (4 splits) and the generic loader accepts.

Views: every fourth projection case and the 3-row expert case are sent again
as a strided view, cycling through a reversed and padded row-major layout, a
column-major layout and an every-other-element layout, stored as f16 or as
f32 values that round to the same f16.  Each view is gathered on the CPU
first and checked against the logical rows.

The generic checkpoint is the same files declared model_type llama: every
metal-checkpoint-linear case again as metal-exl3-linear, and the wide
projection.  Invalid requests: an empty batch, a missing prefix, the refused
geometry, a partial row, the mismatched expert, the direct op on the generic
checkpoint and a view of the wrong width.

Bundle checkpoints (model_type qwen3_5_moe, seed GROUP_SEED): for each K and
cb, 2 + i % 3 projections of input (384, 1536, 4096)[(K + 2 cb) % 3] and
columns 128 (1 + (3 j + K + cb) % 8), scale storage (BF16, F32, F16)[(K + cb)
% 3], bias on members with (i + j) odd, I16 / U16 alternating; two wide dense
bundles (4096 -> 14336 x 2 at K3 MCG, 2048 -> 2048 + 512 + 512 at K4), a
mixed-codebook and a mixed-K pair, a single and a repeated projection, and a
reversed f16 view and a stride-3 f32 view of one row.  Invalid bundle
requests: no prefixes, a missing member, an empty or overlong row, a missing
second member and members of two input widths.

The reference's expected words come from its MLX build, which cannot run
here.  Each output is compared bit for bit with the library's own API on the
same checkpoint (Exl3Linear.from_checkpoint(...).forward, swiglu, Exl3Group)
and, within the linear tolerance, with the oracle on the loader-rounded
weights; bundle outputs are also compared with the mlx-checkpoint-group op.
"""

from __future__ import annotations

import json
from dataclasses import dataclass

import numpy as np
import pytest

import oracle
from codec_client import run
from mlxl3_amd import synth

pytestmark = pytest.mark.gpu

SEED = 31013
GROUP_SEED = 47711
WIDTHS = (256, 1152, 3072, 640, 5120)
SCALES = ("F16", "BF16", "F32")

TOL_REL = 1e-3
TOL_ULP = 2
CHAIN_TOL_REL = 5e-3


def check(y, ref, label, tol=TOL_REL, ulp=TOL_ULP):
    y = np.asarray(y, np.float64)
    r = np.asarray(ref, np.float64)
    rel = np.linalg.norm(y - r) / np.linalg.norm(r)
    ulps = np.abs(y - r).max() / float(np.spacing(np.float16(np.abs(r).max())))
    print(f"{label}: rel_l2={rel:.3e} max_abs={ulps:.2f} ulp", flush=True)
    assert rel <= tol and (ulp is None or ulps <= ulp), (label, rel, ulps)


@dataclass
class Spec:
    name: str
    width: int
    cols: int
    k: int
    cb: int
    scale: str = "F16"
    legacy: bool = False
    signed: bool = True
    bias: bool = False


def bf16_bits(v):
    """Round-to-nearest-even bfloat16 bits of float32 values."""
    b = np.asarray(v, np.float32).view(np.uint32)
    return ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(
        np.uint16)


def off_by_a_little(v16):
    """float32 values one f32 step away from each non-zero f16 value (away from
    zero), so a round-to-nearest cast gives the f16 value back; zeros keep
    their sign."""
    v = np.asarray(v16, np.float16).astype(np.float32)
    return np.where(v == 0, v, np.nextafter(v, np.copysign(np.float32(np.inf), v)))


def stored_scale(v16, dtype):
    """(the tensor a checkpoint stores, the f16 values the loader reads back)."""
    if dtype == "BF16":
        bits = bf16_bits(v16.astype(np.float32))
        return ("BF16", bits), (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float16)
    if dtype == "F32":
        return off_by_a_little(v16), v16
    return v16, v16


def projection(seed, tid, spec):
    """The checkpoint tensors of one projection and its loader-rounded
    (trellis, suh, svh, bias, K, codebook) for the oracle."""
    t, suh, svh, bias = synth.linear_layer(seed, tid, spec.width, spec.cols, spec.k, bias=spec.bias)
    tensors = synth.exl3_tensors(spec.name, t, suh, svh, bias=bias, cb=spec.cb,
                                 legacy_names=spec.legacy, signed=spec.signed)
    su, sv = ("su", "sv") if spec.legacy else ("suh", "svh")
    tensors[f"{spec.name}.{su}"], suh_r = stored_scale(suh, spec.scale)
    tensors[f"{spec.name}.{sv}"], svh_r = stored_scale(svh, spec.scale)
    return tensors, (t, suh_r, svh_r, bias, spec.k, spec.cb)


def rows_in(seed, tid, rows, width, edge=False):
    x = (synth.normal(seed, tid, rows * width) * 0.125).astype(np.float16).reshape(rows, width)
    if edge:
        sub = (np.arange(1, width // 9 + 2) * 37 % 1023 + 1).astype(np.float64) * 2.0 ** -24
        x[0, ::9] = (sub[: len(x[0, ::9])] * np.where(np.arange(len(x[0, ::9])) % 2, -1, 1)).astype(
            np.float16)
        x[-1, 4::13] = np.float16(-0.0)
    return x


def words(x):
    return np.ascontiguousarray(x, np.float16).view(np.uint16).ravel().tolist()


def strided_view(x, kind, use_f32):
    """(storage list, layout) of one strided view of the [rows, width] f16
    matrix x, stored as f16 words or as float32 values that round to x."""
    rows, width = x.shape
    if kind == 0:  # reversed in both axes, 2 leading and 3 trailing pad columns
        pitch = width + 5
        backing = np.full((rows, pitch), np.float16(3.5))
        backing[:, 2:2 + width] = x[::-1, ::-1]
        layout = {"shape": [rows, width], "strides": [-pitch, -1],
                  "offset": (rows - 1) * pitch + 1 + width}
    elif kind == 1:  # column-major after 5 pad elements
        backing = np.concatenate([np.full(5, np.float16(-2)), x.T.ravel()])
        layout = {"shape": [rows, width], "strides": [1, rows], "offset": 5}
    else:  # every other element, starting at 1
        backing = np.zeros(2 * rows * width + 1, np.float16)
        backing[1::2] = x.ravel()
        layout = {"shape": [rows, width], "strides": [2 * width, 2], "offset": 1}
    flat = np.asarray(backing, np.float16).ravel()
    idx = (layout["offset"] + np.arange(rows)[:, None] * layout["strides"][0]
           + np.arange(width)[None, :] * layout["strides"][1])
    assert idx.min() >= 0 and idx.max() < flat.size
    if use_f32:
        store = off_by_a_little(flat)
        assert np.array_equal(store[idx].astype(np.float16).view(np.uint16), x.view(np.uint16))
        return {"x_f32": store.tolist(), "x_layout": layout}
    assert np.array_equal(flat[idx].view(np.uint16), x.view(np.uint16))
    return {"x": flat.view(np.uint16).tolist(), "x_layout": layout}


def flash_fixture(root):
    """The projection checkpoint of the case matrix: (cases, views, weights);
    each case carries its logical rows under "_rows" (not sent)."""
    tensors, storage, weights, cases = {}, {}, {}, []
    tid = 0

    def add(spec):
        nonlocal tid
        t, w = projection(SEED, tid, spec)
        tid += 8
        tensors.update(t)
        storage[spec.name] = {"quant_format": "exl3"}
        weights[spec.name] = w

    for k in range(1, 9):
        for cb in range(3):
            i = 3 * (k - 1) + cb
            name = f"proj.k{k}.cb{cb}"
            add(Spec(name, WIDTHS[i % 5], 128 * (1 + k % 3), k, cb, SCALES[(k + cb) % 3],
                     legacy=i % 4 == 2, signed=i % 2 == 0, bias=(i // 2) % 2 == 0))
            rows = 33 if i in (5, 14) else 1 + 5 * i % 4
            x = rows_in(SEED, 1000 + i, rows, WIDTHS[i % 5], edge=i % 6 == 5)
            cases.append({"op": "metal-checkpoint-linear", "prefix": name, "_rows": x})
    for expert, down_out in (("mlp.ok", 512), ("mlp.bad", 384)):
        add(Spec(f"{expert}.gate_proj", 512, 768, 3, 1, "BF16"))
        add(Spec(f"{expert}.up_proj", 512, 768, 5, 0, "F32", legacy=True, signed=False))
        add(Spec(f"{expert}.down_proj", 768, down_out, 2, 2, "F16", bias=True))
    for n, rows in enumerate((1, 3)):
        cases.append({"op": "metal-checkpoint-expert", "prefix": "mlp.ok",
                      "_rows": rows_in(SEED, 2000 + n, rows, 512)})
    add(Spec("wide", 12288, 256, 2, 0))
    synth.write_checkpoint(root, [tensors], storage, model_type="qwen4_exp", bits=None,
                           index=False)
    for c in cases:
        c["path"] = str(root)
    picked = [c for i, c in enumerate(cases[:24]) if i % 4 == 3] + [cases[-1]]
    views = []
    for n, c in enumerate(picked):
        packet = {k: v for k, v in c.items() if k != "_rows"}
        packet.update(strided_view(c["_rows"], n % 3, use_f32=n % 2 == 1))
        views.append((packet, c))
    return cases, views, weights


def send(c):
    return {**{k: v for k, v in c.items() if k != "_rows"}, "x": words(c["_rows"])}


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

    root = tmp_path / "flash"
    cases, views, weights = flash_fixture(root)
    generic = tmp_path / "generic"
    generic.mkdir()
    for f in root.iterdir():
        (generic / f.name).write_bytes(f.read_bytes())
    (generic / "config.json").write_text(json.dumps({"model_type": "llama"}))
    exl3_cases = [{**c, "path": str(generic), "op": "metal-exl3-linear"}
                  for c in cases if c["op"] == "metal-checkpoint-linear"]
    wide_x = rows_in(SEED, 3000, 2, 12288)
    exl3_cases.append({"op": "metal-exl3-linear", "path": str(generic), "prefix": "wide",
                       "_rows": wide_x})
    first = send(cases[0])
    narrow = {**views[0][0], "x_layout": {**views[0][0]["x_layout"]}}
    narrow["x_layout"]["shape"] = [narrow["x_layout"]["shape"][0], 128]
    invalid = [
        ({**first, "x": []}, "invalid Flash projection batch"),
        ({**first, "prefix": "proj.k9.cb0"}, "missing projection trellis"),
        ({**first, "prefix": "wide"}, "unsupported projection geometry/split count"),
        ({**first, "x": first["x"][:-1]}, "input is not a complete row"),
        ({**send(cases[-1]), "prefix": "mlp.bad"}, "incompatible Flash expert projection geometry"),
        ({**send(exl3_cases[0]), "op": "metal-checkpoint-linear"},
         "requires a Flash reference checkpoint"),
        (narrow, "invalid projection view width"),
    ]
    stream = ([r for r, _ in invalid] + [send(c) for c in cases] + [p for p, _ in views]
              + [send(c) for c in exl3_cases])
    replies = run(stream, timeout=300)
    for (req, message), reply in zip(invalid, replies):
        assert message in reply.get("error", ""), (req["prefix"], message, reply)
    replies = replies[len(invalid):]
    ck = mlxl3_amd.Checkpoint(root)
    ckg = mlxl3_amd.Checkpoint(generic)
    n_words = 0
    expected = {}
    for c, reply in zip(cases, replies[:len(cases)]):
        assert "data" in reply, (c["prefix"], reply)
        got = np.asarray(reply["data"], np.uint16)
        prefix, x = c["prefix"], c["_rows"]
        expert = c["op"] == "metal-checkpoint-expert"
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
        expected[(prefix, c["op"], x.shape[0])] = got
        n_words += got.size
    replies = replies[len(cases):]
    for (packet, c), reply in zip(views, replies[:len(views)]):
        key = (c["prefix"], c["op"], c["_rows"].shape[0])
        assert reply == {"data": expected[key].tolist()}, (c["prefix"], packet["x_layout"])
    replies = replies[len(views):]
    for c, reply in zip(exl3_cases, replies):
        assert "data" in reply, (c["prefix"], reply)
        got = np.asarray(reply["data"], np.uint16)
        if c["prefix"] == "wide":
            mine = library_linear(ckg, "wide", wide_x)
            assert np.array_equal(got, mine.view(np.uint16).ravel())
            check(got.view(np.float16), oracle_linear(weights["wide"], wide_x).ravel(),
                  "exl3 wide")
        else:
            key = (c["prefix"], "metal-checkpoint-linear", c["_rows"].shape[0])
            assert np.array_equal(got, expected[key]), c["prefix"]
    print(f"flash replay: {len(cases)} cases, {len(views)} views, {len(exl3_cases)} generic, "
          f"{n_words} words", flush=True)
    ck.close()
    ckg.close()


def bundle(folder, specs, seed, tid):
    tensors, storage = {}, {}
    for n, spec in enumerate(specs):
        tensors.update(projection(seed, tid + 8 * n, spec)[0])
        storage[spec.name] = {"quant_format": "exl3"}
    synth.write_checkpoint(folder, [tensors], storage, model_type="qwen3_5_moe", bits=None,
                           index=False)
    return str(folder)


def group_fixtures(root):
    """The bundle checkpoints of the case matrix: (cases, expected grouped
    flags); each case carries its logical row under "_rows"."""
    cases, flags = [], []
    tid = 0

    def add(name, specs, grouped, prefixes=None):
        nonlocal tid
        path = bundle(root / name, specs, GROUP_SEED, tid)
        x = rows_in(GROUP_SEED, 5000 + tid, 1, specs[0].width)
        tid += 64
        cases.append({"op": "metal-checkpoint-group", "path": path,
                      "prefixes": prefixes or [s.name for s in specs], "_rows": x})
        flags.append(grouped)

    for k in range(1, 9):
        for cb in range(3):
            i = 3 * (k - 1) + cb
            width = (384, 1536, 4096)[(k + 2 * cb) % 3]
            specs = [Spec(f"q{j}", width, 128 * (1 + (3 * j + k + cb) % 8), k, cb,
                          ("BF16", "F32", "F16")[(k + cb) % 3], signed=j % 2 == 0,
                          bias=(i + j) % 2 == 1, legacy=j == 1 and i % 5 == 0)
                     for j in range(2 + i % 3)]
            add(f"k{k}-cb{cb}", specs, k != 7)
    add("dense-mlp", [Spec(f"q{j}", 4096, 14336, 3, 1) for j in range(2)], True)
    add("dense-qkv", [Spec("q0", 2048, 2048, 4, 0, "BF16"), Spec("q1", 2048, 512, 4, 0, "BF16"),
                      Spec("q2", 2048, 512, 4, 0, "BF16")], True)
    add("mixed-cb", [Spec("q0", 1024, 256, 2, 0), Spec("q1", 1024, 384, 2, 2)], False)
    add("mixed-k", [Spec("q0", 1024, 128, 3, 1), Spec("q1", 1024, 128, 4, 1)], False)
    cases.append({**cases[0], "prefixes": ["q0"]})
    flags.append(False)
    cases.append({**cases[1], "prefixes": ["q1", "q1"]})
    flags.append(True)
    for n, base in enumerate((0, 4)):
        x = cases[base]["_rows"][0]
        if n == 0:  # reversed, f16
            backing = np.concatenate([x[::-1], np.zeros(3, np.float16)])
            view = {"x": backing.view(np.uint16).tolist(),
                    "x_layout": {"shape": [1, x.size], "strides": [x.size, -1],
                                 "offset": x.size - 1}}
        else:  # every third element, f32
            backing = np.full(3 * x.size + 2, np.float32(9.0))
            backing[2::3] = off_by_a_little(x)
            view = {"x_f32": backing.tolist(),
                    "x_layout": {"shape": [1, x.size], "strides": [3 * x.size, 3], "offset": 2}}
        cases.append({**cases[base], **view})
        flags.append(flags[base])
    return cases, flags


def test_projection_group_replay(tmp_path):
    import mlxl3_amd

    cases, flags = group_fixtures(tmp_path)
    first = send(cases[0])
    two_widths = bundle(tmp_path / "two-widths", [Spec("q0", 512, 128, 2, 0),
                                                  Spec("q1", 1024, 128, 2, 0)], GROUP_SEED, 9000)
    invalid = [
        ({**first, "prefixes": []}, "empty projection bundle"),
        ({**first, "prefixes": ["missing"]}, "missing projection trellis"),
        ({**first, "x": []}, "invalid grouped input row length"),
        ({**first, "x": first["x"] + [0]}, "invalid grouped input row length"),
        ({**first, "prefixes": ["q0", "missing"]}, "missing projection trellis"),
        ({**first, "path": two_widths, "prefixes": ["q0", "q1"]},
         "projection bundle requires one input width"),
    ]
    packets = [c if "x_layout" in c else send(c) for c in cases]
    packets = [{k: v for k, v in p.items() if k != "_rows"} for p in packets]
    stock = [{**{k: v for k, v in send(c).items() if k not in ("x_layout", "x_f32")},
              "op": "mlx-checkpoint-group"} for c in cases]
    native = run([r for r, _ in invalid] + packets + [packets[-1]], timeout=300)
    refs = run(stock, timeout=300)
    for (req, message), reply in zip(invalid, native):
        assert message in reply.get("error", ""), (req["prefixes"], message, reply)
    native = native[len(invalid):]
    assert native[-1] == native[-2]
    compared = 0
    for c, want, got in zip(cases, refs, native[:-1]):
        assert "data" in want and "data" in got, (c["path"], want, got)
        want, got = want["data"], got["data"]
        assert type(got["grouped"]) is bool and got["grouped"] == want["grouped"], c["path"]
        assert len(got["outputs"]) == len(want["outputs"]) == len(c["prefixes"])
        ck = mlxl3_amd.Checkpoint(c["path"])
        mine = library_bundle(ck, c["prefixes"], c["_rows"], got["grouped"])
        for prefix, a, b, m in zip(c["prefixes"], got["outputs"], want["outputs"], mine):
            a, b = np.asarray(a, np.uint16), np.asarray(b, np.uint16)
            assert np.array_equal(a, b), (c["path"], prefix)
            assert np.isfinite(a.view(np.float16)).all() and np.any(a != 0)
            assert np.array_equal(a, m.view(np.uint16).ravel()), (c["path"], prefix)
            compared += a.size
        ck.close()
    # grouped exactly when two or more projections share K (not 7) and codebook
    assert [g["data"]["grouped"] for g in native[:-1]] == flags
    print(f"group replay: {len(cases)} cases, {compared} words", flush=True)
