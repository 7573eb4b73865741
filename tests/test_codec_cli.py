"""The codec JSON-lines driver's host operations and error protocol (no GPU):
codec_loop, native/src/main.rs:286-1360.  pack and permutation run on the host
and are checked against the oracle and the reference's golden packed vectors;
every malformed request gets one {"error": ...} line and the stream goes on."""

import json

import numpy as np
import pytest

import oracle
from codec_client import CODEC, run

pytestmark = pytest.mark.skipif(not CODEC.exists(), reason="codec driver not built")


def test_permutation_matches_oracle():
    (row,) = run([{"op": "permutation"}])
    assert row == {"data": oracle.permutation().tolist()}


def test_pack_golden_and_oracle(golden):
    sums = json.loads((golden / "quantizer" / "checksums.json").read_text())
    reqs, want = [], []
    for name in sorted(sums):
        if not name.endswith("-states.u16"):
            continue
        _, k, cb, _ = name.split("-")
        states = np.fromfile(golden / "quantizer" / name, dtype="<u2")
        packed = np.fromfile(golden / "quantizer" / name.replace("states", "packed"), dtype="<u2")
        reqs.append({"op": "pack", "k": int(k), "mode": int(cb), "data": states.tolist()})
        want.append(packed.tolist())
    rng = np.random.default_rng(3)
    for k in range(1, 9):
        states = rng.integers(0, 1 << 16, size=512, dtype=np.uint16)
        reqs.append({"op": "pack", "k": k, "data": states.tolist()})
        want.append(oracle.pack(states, k).ravel().tolist())
    rows = run(reqs)
    assert len(want) >= 8 + 8
    for row, w in zip(rows, want):
        assert row == {"data": w}


@pytest.mark.parametrize(
    "req, message",
    [
        ({"op": "pack", "k": 0}, "K must be in 1..=8, got 0"),
        ({"op": "pack", "k": 9, "data": []}, "K must be in 1..=8, got 9"),
        ({"op": "pack", "k": 3, "data": [1] * 255}, "encoded length must be a multiple of 256"),
        ({"op": "unpack", "k": 2, "data": [1] * 31}, "packed length is not a whole tile"),
        ({"op": "metal-decode", "k": 0, "data": []}, "K must be in 1..=8, got 0"),
        ({"op": "metal-pack", "k": 9, "data": []}, "K must be in 1..=8, got 9"),
        ({"op": "metal-pack", "k": 2, "data": [0] * 255}, "expected whole 256-state tiles"),
        ({"op": "metal-decode", "k": 2, "data": [0] * 33}, "expected whole packed tiles"),
        ({"op": "metal-qmv", "k": 2, "x": [0] * 15, "cols": 16, "data": []},
         "expected positive 16-aligned dimensions"),
        ({"op": "metal-qmv", "k": 2, "x": [0] * 16, "cols": 16, "data": [0] * 31},
         "invalid trellis size or Metal index overflow"),
        ({"op": "metal-swiglu", "x": [1, 2], "data": [1]}, "invalid SwiGLU input extents"),
        # the invalid requests of the reference's tests/physical_prepare128.py
        ({"op": "metal-prepare128", "cols": 127, "x": [0] * 127, "data": [0] * 127},
         "expected complete 128-aligned rows"),
        ({"op": "metal-prepare128", "cols": 128, "x": [0] * 128, "data": [0] * 127},
         "expected complete 128-aligned rows"),
        ({"op": "metal-prepare128", "cols": 128, "x": [0] * 127, "data": [0] * 128},
         "expected complete 128-aligned rows"),
        ({"op": "metal-prepare128", "cols": 0, "x": [], "data": []},
         "expected complete 128-aligned rows"),
        ({"op": "mlx-linear", "k": 2, "suh": [], "x": [1]}, "invalid linear input rows"),
        # the rejected requests of main.rs:5670-5680 (routes checked before any GPU
        # or checkpoint work), then a valid route with a missing bank
        ({"op": "mlx-switch", "key_heads": 2, "cols": 128, "top_k": 1}, "invalid SwitchGLU routes"),
        ({"op": "mlx-switch", "key_heads": 2, "cols": 128, "selected": [2]},
         "invalid SwitchGLU routes"),
        ({"op": "mlx-switch", "key_heads": 2, "cols": 128, "selected": [0, 1, 0], "top_k": 2},
         "invalid SwitchGLU routes"),
        ({"op": "mlx-checkpoint-switch", "key_heads": 256, "selected": [256], "x": [0],
          "path": "/missing"}, "invalid checkpoint SwitchGLU routes"),
        ({"op": "mlx-checkpoint-switch", "key_heads": 256, "x": [0], "path": "/missing"},
         "invalid checkpoint SwitchGLU routes"),
        ({"op": "mlx-switch", "key_heads": 2, "cols": 128, "selected": [1], "x": [0] * 128},
         "tensor byte count does not match shape and dtype"),
        ({"op": "mlx-swiglu-prepare", "cols": 128, "suh": [0] * 256, "selected": [1]},
         "invalid SwiGLU routes"),
        ({"op": "mlx-swiglu-prepare", "cols": 0, "selected": [0]}, "invalid gate/up width"),
        ({"op": "mlx-swiglu-prepare", "cols": 128, "selected": [1], "suh": [0] * 512},
         "tensor byte count does not match shape and dtype"),
        ({"op": "mlx-expert-reduce", "cols": 100, "beta": [0]}, "invalid expert reduction dimensions"),
        ({"op": "mlx-expert-reduce", "cols": 128, "beta": [0], "state": [0.5] * 127},
         "tensor byte count does not match shape and dtype"),
        ({"op": "mlx-switch", "key_heads": 2, "cols": 128, "selected": [1], "x": [0] * 100},
         "invalid SwitchGLU layout"),
        ({"op": "mlx-switch", "key_heads": 2, "cols": 128, "selected": [1], "x": [0] * 128,
          "k": 7}, "invalid SwitchGLU layout"),
        ({"op": "mlx-group", "k": 2, "widths": []}, "missing group widths"),
        ({"op": "mlx-group", "k": 7, "widths": [128, 128], "suh": [0] * 256, "x": [0] * 128},
         "unsupported group"),
        ({"op": "codebook", "mode": 3, "data": [1]}, "invalid EXL3 codebook 3"),
        ({"op": "unpack", "mode": 7, "k": 0}, "invalid EXL3 codebook 7"),
        ({"op": "mlx-gdn"}, "unknown or unavailable codec operation mlx-gdn"),
        ({"op": "pack", "k": 2, "data": [70000] * 256}, "invalid codec request"),
        ({"op": "pack", "k": -1}, "invalid codec request"),
        ({"k": 2}, "invalid codec request"),
    ],
)
def test_errors_are_lines(req, message):
    rows = run([req, {"op": "permutation"}])
    assert list(rows[0]) == ["error"] and message in rows[0]["error"], rows[0]
    assert "data" in rows[1]  # the stream continues


def test_prepare128_empty_batch_needs_no_gpu():
    # physical_prepare128.py: an empty batch of a valid width answers [] (and
    # prepare128_blocks(0, 128, 0) == Some(0), contracts.rs:2163)
    (row,) = run([{"op": "metal-prepare128", "cols": 128, "x": [], "data": []}])
    assert row == {"data": []}


def test_malformed_lines_and_defaults():
    import subprocess

    res = subprocess.run([str(CODEC)], input='not json\n[1]\n{"op": "pack", "data": []}\n',
                         text=True, capture_output=True, check=True, timeout=60)
    rows = [json.loads(line) for line in res.stdout.splitlines()]
    assert "invalid codec request" in rows[0]["error"]
    assert "invalid codec request" in rows[1]["error"]
    assert rows[2] == {"data": []}  # default k = 4 is valid, nothing to pack
    bad = subprocess.run([str(CODEC), "serve"], capture_output=True, text=True, timeout=60)
    assert bad.returncode == 2


def test_prepare_view_rejections_of_the_reference_harness():
    """The rejected metal-prepare-view requests of the reference's
    tests/physical_prepare128.py, answered before any GPU work, and its empty
    view starting one element past the storage."""
    view = {"shape": [1, 128], "strides": [0, 0], "offset": 0}
    zero = {"op": "metal-prepare-view", "x": [0], "data": [0], "x_layout": view,
            "scale_layout": view}
    cases = [({"x_layout": {**view, "strides": [0, -1]}}, "outside initialized storage"),
             ({"scale_layout": {**view, "strides": [0, 2 ** 63 - 1]}}, "outside initialized storage"),
             ({"x_layout": {**view, "offset": -1}}, "outside initialized storage"),
             ({"x_layout": {**view, "shape": [2, 128]}}, "invalid H128 view shape"),
             ({"x_f32": [0]}, "conflicting input buffer dtypes"),
             ({"x_layout": None}, "missing input matrix layout"),
             ({"scale_layout": None}, "missing scale matrix layout"),
             ({"x_layout": {**view, "shape": [1, 127]}, "scale_layout": {**view, "shape": [1, 127]}},
              "128-aligned"),
             ({"x_layout": {**view, "shape": [2 ** 31, 128]},
               "scale_layout": {**view, "shape": [2 ** 31, 128]}}, "size overflow")]
    one_past = {**view, "shape": [0, 128], "offset": 1}
    rows = run([{**zero, **f} for f, _ in cases] + [{**zero, "x_layout": one_past,
                                                     "scale_layout": one_past}])
    for (_, msg), row in zip(cases, rows):
        assert msg in row.get("error", ""), (msg, row)
    assert rows[-1] == {"data": []}


def _bank_checkpoint(tmp_path):
    """A synthetic checkpoint (host files only) with a 2-expert 128->128 bank and
    two projections of different input widths."""
    from mlxl3_amd import synth

    tensors = {}
    for e in range(2):
        for p, (i, o) in zip(("gate_proj", "up_proj", "down_proj"), ((128, 128), (128, 128), (128, 128))):
            t, suh, svh, _ = synth.linear_layer(7, e * 16 + len(p), i, o, 2)
            tensors.update(synth.exl3_tensors(f"m.experts.{e}.{p}", t, suh, svh))
    for name, (i, o) in (("q", (256, 128)), ("k", (128, 128))):
        t, suh, svh, _ = synth.linear_layer(9, len(name), i, o, 2)
        tensors.update(synth.exl3_tensors(f"m.attn.{name}", t, suh, svh))
    storage = {p: {"quant_format": "exl3"} for p in ("m.attn.q", "m.attn.k")}
    return synth.write_checkpoint(tmp_path / "ckpt", [tensors], storage)


def test_checkpoint_ops_check_input_widths_before_any_upload(tmp_path):
    """Exl3SwitchGlu::forward rejects a row that is not the bank's input width
    (moe.rs:911-918) and each projection's forward rejects a row that is not its
    own width (linear.rs:739-743, Exl3Group::forward :2388-2391): the driver
    answers with those errors before any device allocation, so a short x never
    reaches a kernel."""
    root = str(_bank_checkpoint(tmp_path))
    rows = run([
        {"op": "mlx-checkpoint-switch", "path": root, "prefix": "m.experts", "key_heads": 2,
         "selected": [0], "beta": [15360], "x": [0] * 64},
        {"op": "mlx-checkpoint-group", "path": root, "prefixes": ["m.attn.q", "m.attn.k"],
         "x": [0] * 128},
        {"op": "mlx-checkpoint-group", "path": root, "prefixes": ["m.attn.k", "m.attn.q"],
         "x": [0] * 128},
        {"op": "permutation"},
    ])
    assert rows[0] == {"error": "invalid SwitchGLU input/routes"}, rows[0]
    # widths 256 and 128 cannot group: each projection checks its own width
    assert rows[1] == {"error": "invalid EXL3 linear input for 256 inputs"}, rows[1]
    assert rows[2] == {"error": "invalid EXL3 linear input for 256 inputs"}, rows[2]
    assert "data" in rows[3]
