"""Checkpoint inspection and loader validation (host code, no GPU).

Covers exl3_checkpoint_open (checkpoint::inspect, native/src/checkpoint.rs:197-330,
read_header :38-93), the tensor records and payload reads, the f16 conversion the
loaders apply (MLX astype(Float16)), and the argument checks of exl3_linear_load
(Exl3Linear::from_checkpoint / new, linear.rs:454-607) and exl3_moe_load
(moe.rs:681-800) that run before anything touches a device.  The error texts are
the reference's (checkpoint.rs, linear.rs, moe.rs); the reference's own tests of
inspection are the Rust unit tests beside it, which build checkpoints the same way
(a temporary directory with config, quantization config, tokenizer and shards).
"""

from __future__ import annotations

import json
import struct

import numpy as np
import pytest

import mlxl3_amd
from mlxl3_amd import synth
from mlxl3_amd import Checkpoint, Exl3Error

pytestmark = pytest.mark.skipif(not mlxl3_amd.LIB_PATH.exists(), reason="library not built")


def _linear_tensors(prefix, in_f=256, out_f=128, k=2, cb=0, seed=1, **kw):
    t, suh, svh, bias = synth.linear_layer(seed, hash(prefix) & 0xFFFF, in_f, out_f, k)
    return synth.exl3_tensors(prefix, t, suh, svh, bias if kw.pop("with_bias", False) else None,
                              cb=cb, **kw)


def _storage(*prefixes, extra=None):
    st = {p: {"quant_format": "exl3"} for p in prefixes}
    st.update(extra or {})
    return st


def _ok_dir(tmp_path, **kw):
    a = _linear_tensors("model.layers.0.mlp.up_proj", with_bias=True)
    b = _linear_tensors("model.layers.0.mlp.down_proj", in_f=128, out_f=256, cb=1, legacy_names=True)
    c = _linear_tensors("model.layers.1.self_attn.q_proj", cb=2, scale_dtype="BF16")
    norm = {"model.norm.weight": np.arange(256, dtype=np.float16)}
    storage = _storage("model.layers.0.mlp.up_proj", "model.layers.0.mlp.down_proj",
                       "model.layers.1.self_attn.q_proj",
                       extra={"model.norm": {"quant_format": "fp16",
                                             "stored_tensors": {"model.norm.weight": {"shape": [256]}}}})
    return synth.write_checkpoint(tmp_path / "ckpt", [{**a, **norm}, {**b, **c}], storage, **kw), (a, b, c, norm)


def _expect(tmp_path, message, status=-1):
    with pytest.raises(Exl3Error) as e:
        Checkpoint(tmp_path)
    assert message in str(e.value), str(e.value)
    assert e.value.status == status
    return str(e.value)


def test_inspect_round_trip(tmp_path):
    root, (a, b, c, norm) = _ok_dir(tmp_path, model_type="qwen3", bits=3.5)
    ck = Checkpoint(root)
    assert ck.path == str(root.resolve())
    assert ck.model_type == "qwen3" and ck.bits == 3.5
    assert ck.modules == sorted(["model.layers.0.mlp.up_proj", "model.layers.0.mlp.down_proj",
                                 "model.layers.1.self_attn.q_proj"])
    assert ck.size_bytes == sum(p.stat().st_size for p in root.iterdir() if p.is_file())
    every = {**a, **b, **c, **norm}
    assert ck.tensor_names == sorted(every)
    for name, value in every.items():
        dtype, arr = value if isinstance(value, tuple) else (synth._ST_DTYPES[value.dtype], value)
        info = ck.info(name)
        assert info.dtype == dtype and info.shape == arr.shape
        assert info.nbytes == arr.nbytes
        # the record's absolute offset addresses the payload in the shard file
        with open(info.shard, "rb") as fh:
            fh.seek(info.offset)
            assert fh.read(info.nbytes) == np.asarray(arr, order="C").tobytes()
        assert ck.read(name).tobytes() == np.asarray(arr, order="C").tobytes()
    assert "model.norm.weight" in ck and "nope" not in ck
    ck.close()


def test_bits_absent_and_single_shard_without_index(tmp_path):
    a = _linear_tensors("p")
    root = synth.write_checkpoint(tmp_path / "c", [a], _storage("p"), bits=None, index=False)
    ck = Checkpoint(root)
    assert ck.bits is None and ck.modules == ["p"] and ck.model_type == "llama"


def test_real_tile_offsets_follow_tensor_layout(golden, tmp_path):
    """The reference's frozen real tiles record each tile's byte offset in its
    shard: offset(t) - offset(0) = t * 16K * 2 for the [in/16][out/16][16K]
    layout.  A shard holding a tensor of the same name, dtype and shape, with
    those tiles at those indices, must hand back the same words through the
    tensor record and read()."""
    for name in ("flash", "qwen-dense", "qwen-moe", "lfm-moe"):
        fix = json.loads((golden / "real_tiles" / f"{name}.json").read_text())
        nr, nc, nw = fix["shape"]
        assert nw == 16 * fix["k"]
        base = fix["tiles"][0]["shard_offset_bytes"]
        rng = np.random.default_rng(len(name))
        words = rng.integers(0, 1 << 16, size=nr * nc * nw, dtype=np.uint16).reshape(nr * nc, nw)
        for tile in fix["tiles"]:
            assert tile["shard_offset_bytes"] - base == tile["tile"] * nw * 2
            words[tile["tile"]] = tile["packed"]
        prefix = fix["tensor"].removesuffix(".trellis")
        tensors = synth.exl3_tensors(prefix, words.reshape(nr, nc, nw), np.ones(nr * 16, np.float16),
                                     np.ones(nc * 16, np.float16), cb=fix["mode"], signed=fix["dtype"] == "I16")
        root = synth.write_checkpoint(tmp_path / name, [tensors], _storage(prefix))
        ck = Checkpoint(root)
        info = ck.info(fix["tensor"])
        assert info.dtype == fix["dtype"] and list(info.shape) == fix["shape"]
        got = ck.read(fix["tensor"]).view(np.uint16).reshape(nr * nc, nw)
        with open(info.shard, "rb") as fh:
            for tile in fix["tiles"]:
                assert got[tile["tile"]].tolist() == tile["packed"]
                fh.seek(info.offset + tile["tile"] * nw * 2)
                assert list(struct.unpack(f"<{nw}H", fh.read(nw * 2))) == tile["packed"]
        # codebook flags: mode 2 <-> .mul1, 1 <-> .mcg, 0 <-> neither (linear.rs:502-508)
        assert (prefix + ".mul1" in ck, prefix + ".mcg" in ck) == (fix["mode"] == 2, fix["mode"] == 1)
        ck.close()


# --- read_header (checkpoint.rs:38-93) ---------------------------------------

def _shard_dir(tmp_path, blob: bytes, extra_tensors=None):
    """A valid directory whose second shard is `blob`."""
    a = _linear_tensors("p")
    root = synth.write_checkpoint(tmp_path / "c", [a], _storage("p"), index=False)
    (root / "model-bad.safetensors").write_bytes(blob)
    return root


def _raw_shard(header: dict | bytes, payload: bytes = b"", length=None) -> bytes:
    text = header if isinstance(header, bytes) else json.dumps(header).encode()
    n = len(text) if length is None else length
    return struct.pack("<Q", n) + text + payload


@pytest.mark.parametrize(
    "blob, message",
    [
        (b"\x01\x02", "missing safetensors header length"),
        (_raw_shard(b"{}", length=10**9), "invalid safetensors header length"),
        (_raw_shard(b"{}", length=100_000_001), "invalid safetensors header length"),
        (_raw_shard(b"{\"a\": "), "invalid safetensors header JSON"),
        (_raw_shard(b"[1, 2]"), "invalid safetensors header JSON"),
        (_raw_shard(b"{} x"), "invalid safetensors header JSON"),
        (_raw_shard({"__metadata__": {"k": 1}}), "invalid safetensors metadata"),
        (_raw_shard({"t": {"dtype": "F16", "shape": [2]}}, b"\0" * 4), "invalid tensor t"),
        (_raw_shard({"t": {"dtype": "F16", "shape": [2], "data_offsets": [0, 4, 8]}}, b"\0" * 4),
         "invalid tensor t"),
        (_raw_shard({"t": {"dtype": "F16", "shape": [2.0], "data_offsets": [0, 4]}}, b"\0" * 4),
         "invalid tensor t"),
        (_raw_shard({"t": {"dtype": "F16", "shape": [-2], "data_offsets": [0, 4]}}, b"\0" * 4),
         "invalid tensor t"),
        (_raw_shard({"t": {"dtype": "Q4", "shape": [2], "data_offsets": [0, 4]}}, b"\0" * 4),
         "unsupported safetensors dtype Q4"),
        (_raw_shard({"t": {"dtype": "F64", "shape": [2**62, 8], "data_offsets": [0, 4]}}, b"\0" * 4),
         "tensor size overflow"),
        (_raw_shard({"t": {"dtype": "F16", "shape": [2], "data_offsets": [0, 6]}}, b"\0" * 6),
         "invalid data range for tensor t"),
        (_raw_shard({"t": {"dtype": "F16", "shape": [2], "data_offsets": [4, 8]}}, b"\0" * 4),
         "invalid data range for tensor t"),
        (_raw_shard({"t": {"dtype": "F16", "shape": [2], "data_offsets": [2, 6]}}, b"\0" * 6),
         "safetensors payload has gaps or overlapping tensors"),
        (_raw_shard({"t": {"dtype": "F16", "shape": [2], "data_offsets": [0, 4]},
                     "u": {"dtype": "F16", "shape": [2], "data_offsets": [2, 6]}}, b"\0" * 6),
         "safetensors payload has gaps or overlapping tensors"),
        (_raw_shard({"t": {"dtype": "F16", "shape": [2], "data_offsets": [0, 4]}}, b"\0" * 6),
         "unclaimed safetensors payload"),
    ],
)
def test_read_header_rejects(tmp_path, blob, message):
    _expect(_shard_dir(tmp_path, blob), message)


def test_read_header_accepts_metadata_scalars_and_empty_tensors(tmp_path):
    text = json.dumps({"__metadata__": {"format": "pt"},
                       "s": {"dtype": "I32", "shape": [], "data_offsets": [0, 4]},
                       "e": {"dtype": "F16", "shape": [0, 3], "data_offsets": [4, 4]},
                       "NAME": {"dtype": "U8", "shape": [1], "data_offsets": [4, 5]}})
    # a raw UTF-8 character and an escaped surrogate pair in one key
    text = text.replace("NAME", "\u00e9\\ud83d\\ude00").encode()
    blob = _raw_shard(text, b"\x07\0\0\0\x09")
    root = _shard_dir(tmp_path, blob)
    ck = Checkpoint(root)
    assert ck.info("s").shape == () and ck.read("s").tolist() == 7
    assert ck.info("e").shape == (0, 3) and ck.info("e").nbytes == 0
    assert ck.read("é\U0001F600").tolist() == [9]


# --- inspect (checkpoint.rs:197-330) ------------------------------------------

def test_inspect_directory_and_config_errors(tmp_path):
    _expect(tmp_path / "missing", "model directory")
    root, _ = _ok_dir(tmp_path)
    (root / "config.json").write_text("[]")
    _expect(root, "model config must be an object")
    (root / "config.json").write_text("{")
    _expect(root, "invalid JSON in")
    (root / "config.json").write_text("{}")
    q = json.loads((root / "quantization_config.json").read_text())
    (root / "quantization_config.json").write_text(json.dumps({**q, "quant_method": "gptq"}))
    _expect(root, "expected quant_method='exl3'")
    (root / "quantization_config.json").write_text(json.dumps({**q, "tensor_storage": []}))
    _expect(root, "invalid EXL3 tensor_storage")
    (root / "quantization_config.json").write_text(json.dumps(q))
    assert Checkpoint(root).model_type == "unknown"


def test_inspect_shard_set_errors(tmp_path):
    a = _linear_tensors("p")
    root = synth.write_checkpoint(tmp_path / "dup", [a, {"p.trellis": a["p.trellis"]}], _storage("p"),
                                  index=False)
    _expect(root, "duplicate tensor p.trellis")
    root = synth.write_checkpoint(tmp_path / "tok", [a], _storage("p"), tokenizer=False)
    _expect(root, "missing tokenizer files; download the complete checkpoint")
    for name in ("tokenizer_config.json", "spm.model", "vocab.json"):
        (root / name).write_text("{}")
        Checkpoint(root).close()
        (root / name).unlink()
    root = synth.write_checkpoint(tmp_path / "none", [], _storage("p"))
    _expect(root, "checkpoint has no safetensors weights")
    # only model*.safetensors are shards (other files are ignored)
    root = synth.write_checkpoint(tmp_path / "other", [a], _storage("p"))
    (root / "extra.safetensors").write_bytes(b"garbage")
    Checkpoint(root).close()


def test_inspect_storage_errors(tmp_path):
    a = _linear_tensors("p")
    norm = {"n.weight": np.zeros(8, np.float16)}

    def check(storage, message, tensors=None):
        root = synth.write_checkpoint(tmp_path / f"s{abs(hash(message)) % 10**8}",
                                      [tensors if tensors is not None else {**a, **norm}], storage)
        return _expect(root, message)

    check(_storage("p", extra={"q": 3}), "invalid tensor_storage entry q")
    check(_storage("p", extra={"n": {"stored_tensors": []}}), "invalid stored_tensors")
    check(_storage("p", extra={"n": {"stored_tensors": {"n.weight": {"shape": "8"}}}}),
          "invalid stored tensor shape")
    check(_storage("p", extra={"n": {"stored_tensors": {"n.bias": {"shape": [8]}}}}), "missing tensor n.bias")
    check(_storage("p", extra={"n": {"stored_tensors": {"n.weight": {"shape": [9]}}}}),
          "invalid shape for tensor n.weight")
    check(_storage("p", "q"), "missing trellis q")
    check({}, "checkpoint contains no EXL3 modules")
    check({"p": {"quant_format": "fp16"}}, "checkpoint contains no EXL3 modules")
    bad = dict(a)
    bad["p.trellis"] = a["p.trellis"].astype(np.float16)
    check(_storage("p"), "invalid EXL3 trellis p", bad)
    bad["p.trellis"] = a["p.trellis"].reshape(16, -1)
    check(_storage("p"), "invalid EXL3 trellis p", bad)
    bad["p.trellis"] = np.zeros((16, 8, 144), np.int16)
    check(_storage("p"), "invalid EXL3 trellis p", bad)
    bad["p.trellis"] = np.zeros((16, 8, 24), np.int16)
    check(_storage("p"), "invalid EXL3 trellis p", bad)
    bad = {k: v for k, v in a.items() if k != "p.svh"}
    check(_storage("p"), "missing scale p.svh", bad)
    bad = dict(a)
    bad["p.suh"] = np.ones(255, np.float16)
    check(_storage("p"), "invalid scale shape p.suh", bad)
    bad["p.suh"] = np.ones(256, np.int16)
    check(_storage("p"), "invalid scale dtype p.suh", bad)


def test_lfm2_moe_expert_bias_alias(tmp_path):
    a = _linear_tensors("p")
    bias = {"model.layers.3.feed_forward.expert_bias": np.zeros(4, np.float32)}
    stored = {"model.layers.3.feed_forward.gate": {
        "stored_tensors": {"model.layers.3.feed_forward.gate.expert_bias": {"shape": [4]}}}}
    root = synth.write_checkpoint(tmp_path / "lfm", [{**a, **bias}], _storage("p", extra=stored),
                                  model_type="lfm2_moe")
    Checkpoint(root).close()
    root = synth.write_checkpoint(tmp_path / "other", [{**a, **bias}], _storage("p", extra=stored))
    _expect(root, "missing tensor model.layers.3.feed_forward.gate.expert_bias")


def test_shard_index_errors(tmp_path):
    root, _ = _ok_dir(tmp_path)
    index = json.loads((root / "model.safetensors.index.json").read_text())
    wm = index["weight_map"]
    shards = sorted(set(wm.values()))

    def write(m):
        (root / "model.safetensors.index.json").write_text(json.dumps({"weight_map": m}))

    write({**wm, "model.norm.weight": shards[1]})
    _expect(root, "tensor model.norm.weight is in the wrong shard")
    write({**wm, "ghost": shards[0]})
    _expect(root, "missing indexed tensor ghost")
    write({**wm, "model.norm.weight": "sub/" + shards[0]})
    _expect(root, "invalid shard path")
    write({**wm, "model.norm.weight": 3})
    _expect(root, "invalid shard name")
    (root / "model.safetensors.index.json").write_text(json.dumps({"weight_map": []}))
    _expect(root, "invalid shard index")
    write(wm)
    Checkpoint(root).close()


def test_json_reader_strictness(tmp_path):
    """The header reader is strict JSON: what serde_json refuses is refused."""
    good = {"t": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}
    for text in (b'{"t": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1],}}',  # trailing comma
                 b"{'t': 1}", b'{"t": NaN}', b'{"a": "\\x41"}', b'{"a": "\\ud800"}',
                 b'{"a": "\x01"}', b'{"a": 01}', b'{"a": 1.}', b'{"a": "\xff"}',
                 b"[" * 200 + b"]" * 200):
        _expect(_shard_dir(tmp_path / str(abs(hash(text))), _raw_shard(text, b"\0")),
                "invalid safetensors header JSON")
    # whitespace padding and escapes are fine; a repeated key keeps its last value
    text = b' \n{"t": {"dtype": "F16", "shape": [9], "data_offsets": [0, 1]}, "t": ' + \
        json.dumps(good["t"]).encode() + b"}\t  "
    Checkpoint(_shard_dir(tmp_path / "ok", _raw_shard(text, b"\0"))).close()


def test_read_checks_and_truncation(tmp_path):
    root, _ = _ok_dir(tmp_path)
    ck = Checkpoint(root)
    lib = mlxl3_amd.load_library()
    buf = np.zeros(8, np.uint8)
    assert lib.exl3_checkpoint_read(ck.handle, b"model.norm.weight", buf.ctypes.data, 8) == -1
    assert "has 512 bytes, buffer has 8" in lib.exl3_last_error().decode()
    assert lib.exl3_checkpoint_read(ck.handle, b"ghost", buf.ctypes.data, 8) == -1
    assert b"missing tensor ghost" in lib.exl3_last_error()
    shard = ck.info("model.norm.weight").shard
    # payloads are read from the descriptor opened at inspection
    with open(shard, "r+b") as fh:
        fh.truncate(100)
    with pytest.raises(Exl3Error, match="checkpoint was truncated after inspection"):
        ck.read("model.norm.weight")


def test_read_f16_matches_numpy_rounding(tmp_path):
    """exl3_checkpoint_read_f16 rounds like numpy's IEEE f32 -> f16 cast (nearest
    even, gradual underflow, overflow to inf); bf16 inputs are exact in f32, so
    every one of the 65536 bf16 patterns checks the same single rounding."""
    rng = np.random.default_rng(5)
    special = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 65536.0, 1e30, -1e30,
                        np.inf, -np.inf, 2.0**-14, 2.0**-24, 2.0**-25, 2.0**-25 * 1.0000001,
                        2.0**-26, 3 * 2.0**-25, 2.0**-24 * 1.5, 2.0**-24 * 2.5, 1e-45,
                        1 + 2.0**-11, 1 + 3 * 2.0**-11, 1 + 2.0**-11 + 2.0**-23], np.float32)
    bits = rng.integers(0, 1 << 32, size=1 << 18, dtype=np.uint64).astype(np.uint32)
    near = (np.arange(-2000, 2000, dtype=np.int64) + 0x477FF000).astype(np.uint32)
    sub = (np.arange(0, 1 << 16, dtype=np.int64) * 0x80 + 0x33000000).astype(np.uint32)
    f32 = np.concatenate([special, bits.view(np.float32), near.view(np.float32), sub.view(np.float32)])
    bf = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    with np.errstate(over="ignore"):
        h = f32.astype(np.float16)
    root = synth.write_checkpoint(tmp_path / "c", [{**_linear_tensors("p"), "x": f32, "b": ("BF16", bf),
                                                    "h": h}], _storage("p"))
    ck = Checkpoint(root)
    with np.errstate(over="ignore", invalid="ignore"):
        for name, ref in (("x", f32.astype(np.float16)),
                          ("b", (bf.astype(np.uint32) << 16).view(np.float32).astype(np.float16)),
                          ("h", f32.astype(np.float16))):
            got = ck.read_f16(name)
            nan = np.isnan(ref)
            assert np.array_equal(np.isnan(got), nan), name
            assert np.array_equal(got[~nan].view(np.uint16), ref[~nan].view(np.uint16)), name
    with pytest.raises(Exl3Error, match="cannot convert I16 tensor p.trellis to F16"):
        ck.read_f16("p.trellis")


# --- loader validation before any device work ----------------------------------

def _load_linear_error(ck, prefix):
    lib = mlxl3_amd.load_library()
    import ctypes

    h = ctypes.c_void_p()
    status = lib.exl3_linear_load(ck.handle, prefix.encode(), ctypes.byref(h))
    assert status != 0 and not h.value
    return status, lib.exl3_last_error().decode()


def test_linear_load_validation(tmp_path):
    t16 = np.zeros((16, 8, 32), np.int16)
    ones = lambda n: np.ones(n, np.float16)  # noqa: E731
    tensors = {
        **_linear_tensors("p"),
        # not exl3 modules in tensor_storage, so inspection leaves them alone
        "k0.trellis": np.zeros((16, 8, 8), np.int16), "k0.suh": ones(256), "k0.svh": ones(128),
        "k9.trellis": np.zeros((16, 8, 144), np.int16), "k9.suh": ones(256), "k9.svh": ones(128),
        "r2.trellis": np.zeros((16, 128), np.int16), "r2.suh": ones(256), "r2.svh": ones(128),
        "al.trellis": np.zeros((9, 8, 32), np.int16), "al.suh": ones(144), "al.svh": ones(128),
        "sc.trellis": t16, "sc.suh": ones(128), "sc.svh": ones(128),
        "bi.trellis": t16, "bi.suh": ones(256), "bi.svh": ones(128), "bi.bias": ones(64),
        "f16.trellis": t16.astype(np.float16), "f16.suh": ones(256), "f16.svh": ones(128),
        "u64.trellis": t16.astype(np.uint64), "u64.suh": ones(256), "u64.svh": ones(128),
        "nos.trellis": t16,
        "sca.trellis": t16, "sca.suh": np.ones(256, np.int64), "sca.svh": ones(128),
    }
    root = synth.write_checkpoint(tmp_path / "c", [tensors], _storage("p"))
    ck = Checkpoint(root)
    for prefix, message in [
        ("ghost", "missing tensor ghost.trellis"),
        ("k0", "K must be in 1..=8, got 0"),
        ("k9", "K must be in 1..=8, got 9"),
        ("r2", "invalid trellis shape"),
        ("al", "public EXL3 projections require 128-aligned dimensions"),
        ("sc", "EXL3 scales have wrong dimensions"),
        ("bi", "EXL3 bias has wrong dimensions"),
        ("f16", "EXL3 trellis must contain 16-bit integers"),
        ("u64", "unsupported model tensor dtype U64 (u64.trellis)"),
        ("nos", "missing tensor nos.su"),
        ("sca", "unsupported model tensor dtype I64 (sca.suh)"),
    ]:
        status, msg = _load_linear_error(ck, prefix)
        assert message in msg, (prefix, msg)
        assert status == -1


def _expert_bank(prefix, experts, in_f, hidden, k, cb=0, names=("gate_proj", "up_proj", "down_proj")):
    out = {}
    for e in range(experts):
        for p, (i, o) in zip(names, ((in_f, hidden), (in_f, hidden), (hidden, in_f))):
            t, suh, svh, _ = synth.linear_layer(7, e * 16 + len(p), i, o, k)
            out.update(synth.exl3_tensors(f"{prefix}.{e}.{p}", t, suh, svh, cb=cb))
    return out


def _load_moe_error(ck, prefix, experts, top_k, names=(None, None, None)):
    import ctypes

    lib = mlxl3_amd.load_library()
    h = ctypes.c_void_p()
    enc = [n.encode() if n else None for n in names]
    status = lib.exl3_moe_load(ck.handle, prefix.encode(), experts, top_k, *enc, ctypes.byref(h))
    assert status != 0 and not h.value
    return status, lib.exl3_last_error().decode()


def test_moe_load_validation(tmp_path):
    bank = _expert_bank("m.experts", 3, 128, 128, 2)
    mixed_k = _expert_bank("k.experts", 2, 128, 128, 2)
    mixed_k.update(_expert_bank("kk", 1, 128, 128, 3))
    mixed_k = {n.replace("kk.0.", "k.experts.1."): v for n, v in mixed_k.items()}
    mixed_cb = _expert_bank("c.experts", 2, 128, 128, 2)
    mixed_cb["c.experts.1.up_proj.mcg"] = np.array(1, np.int32).reshape(())
    shape = _expert_bank("s.experts", 2, 128, 128, 2)
    t, suh, svh, _ = synth.linear_layer(9, 1, 256, 128, 2)
    shape.update(synth.exl3_tensors("s.experts.1.gate_proj", t, suh, svh))
    scale = _expert_bank("f.experts", 2, 128, 128, 2)
    scale["f.experts.1.down_proj.svh"] = scale["f.experts.1.down_proj.svh"].astype(np.float32)
    bad_dtype = _expert_bank("d.experts", 1, 128, 128, 2)
    bad_dtype["d.experts.0.up_proj.trellis"] = bad_dtype["d.experts.0.up_proj.trellis"].astype(np.int32)
    k7 = _expert_bank("x.experts", 1, 128, 128, 7)
    everything = {**bank, **mixed_k, **mixed_cb, **shape, **scale, **bad_dtype, **k7,
                  **_linear_tensors("p")}
    root = synth.write_checkpoint(tmp_path / "c", [everything], _storage("p"))
    ck = Checkpoint(root)
    for args, message, status in [
        (("m.experts", 0, 1), "invalid expert count or incomplete expert bank", -1),
        (("m.experts", 3, 4), "invalid expert count or incomplete expert bank", -1),
        (("m.experts", 10**6, 1), "invalid expert count or incomplete expert bank", -1),
        (("m.experts", 4, 2), "missing expert trellis m.experts.3.gate_proj", -1),
        (("k.experts", 2, 1), "mixed expert bit widths", -1),
        (("c.experts", 2, 1), "mixed expert codebooks", -1),
        (("s.experts", 2, 1), "SwitchGLU trellis/scales disagree", -1),
        (("f.experts", 2, 1), "this build loads F16 banks", -4),
        (("d.experts", 1, 1), "d.experts.0.up_proj: expert trellis must contain 16-bit integers", -1),
        (("x.experts", 1, 1), "invalid or overflowing SwitchGLU dimensions", -1),
    ]:
        got_status, msg = _load_moe_error(ck, *args)
        assert message in msg, (args, msg)
        assert got_status == status, (args, got_status)
    status, msg = _load_moe_error(ck, "m.experts", 3, 1, ("w1", "w3", "w2"))
    assert "missing expert trellis m.experts.0.w1" in msg
