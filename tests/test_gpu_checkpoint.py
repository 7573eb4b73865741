"""Checkpoint-loaded EXL3 projections and expert banks on the GPU.

exl3_linear_load (Exl3Linear::from_checkpoint, native/src/linear.rs:454-575) and
exl3_moe_load (Exl3SwitchGlu::from_checkpoint_names, native/src/moe.rs:681-800)
against:
* the same weights handed to exl3_linear_create / exl3_moe_create by the caller,
  with the scales rounded to f16 by numpy and the expert bank concatenated by
  numpy (an assembly independent of the loader's): bit-exact outputs;
* the CPU oracle on those numpy-prepared weights: the tolerances of
  test_gpu_linear.py / test_gpu_moe.py (rel L2 <= 1e-3, max-abs <= 2 f16 ulp of
  max|y| for projections; rel L2 <= 1e-3, max-abs <= 1e-2 rms for banks);
* the reference's frozen real checkpoint tiles: shards that hold each fixture's
  tensor at its real name, dtype and shape (tiles placed at their recorded
  indices) decode, through the loader's read path, to the recorded states and
  f16 values bit for bit.
"""

from __future__ import annotations

import json

import numpy as np
import pytest

import oracle
from mlxl3_amd import synth

pytestmark = pytest.mark.gpu

TOL_REL = 1e-3
TOL_ULP = 2
MOE_TOL_RMS = 1e-2


def torch_mod():
    import torch

    return torch


def dev(a):
    torch = torch_mod()
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint32:
        a = a.astype(np.int32)
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def f16_of(value):
    """numpy's f16 rounding of a stored scale (F16 / BF16 bits / F32)."""
    if isinstance(value, tuple):
        return (value[1].astype(np.uint32) << 16).view(np.float32).astype(np.float16)
    return np.asarray(value).astype(np.float16)


def check_linear(y, ref, label):
    y = np.asarray(y, np.float64)
    r = np.asarray(ref, np.float64)
    rel = np.linalg.norm(y - r) / np.linalg.norm(r)
    ulps = np.abs(y - r).max() / float(np.spacing(np.float16(np.abs(r).max())))
    print(f"{label}: rel_l2={rel:.3e} max_abs={ulps:.2f} ulp", flush=True)
    assert rel <= TOL_REL and ulps <= TOL_ULP, (label, rel, ulps)


@pytest.mark.parametrize(
    "k, cb, legacy, scale_dtype, bias, signed",
    [
        (2, 0, False, "F16", False, True),
        (3, 1, True, "BF16", True, True),
        (4, 2, False, "F32", True, False),
        (8, 1, True, "F32", False, False),
    ],
)
def test_linear_load_equals_create(tmp_path, k, cb, legacy, scale_dtype, bias, signed):
    import mlxl3_amd

    torch = torch_mod()
    n_in, n_out = 512, 384
    print(f"linear load k={k} cb={cb} legacy={legacy} scales={scale_dtype} bias={bias}", flush=True)
    tr, suh, svh, b = synth.linear_layer(60 + k, 10, n_in, n_out, k, bias=True)
    # scales with more precision than f16, so the rounding is exercised
    suh32 = suh.astype(np.float32) * np.float32(1.0 + 2.0**-12)
    svh32 = svh.astype(np.float32) * np.float32(1.0 - 2.0**-13)
    tensors = synth.exl3_tensors("blk.proj", tr, suh32, svh32, cb=cb, legacy_names=legacy,
                                 scale_dtype=scale_dtype, signed=signed)
    if bias:
        tensors["blk.proj.bias"] = b.astype(np.float32) * np.float32(1.0 + 2.0**-11)
    root = synth.write_checkpoint(tmp_path / "c", [tensors], {"blk.proj": {"quant_format": "exl3"}})
    ck = mlxl3_amd.Checkpoint(root)
    loaded = mlxl3_amd.Exl3Linear.from_checkpoint(ck, "blk.proj")
    assert (loaded.in_features, loaded.out_features, loaded.k, loaded.cb) == (n_in, n_out, k, cb)
    su, sv = ("su", "sv") if legacy else ("suh", "svh")
    s16 = f16_of(tensors[f"blk.proj.{su}"])
    v16 = f16_of(tensors[f"blk.proj.{sv}"])
    b16 = f16_of(tensors["blk.proj.bias"]) if bias else None
    made = mlxl3_amd.Exl3Linear(dev(tr), dev(s16), dev(v16), None if b16 is None else dev(b16), k, cb)
    for rows in (1, 7, 40):
        x = synth.activations(70 + rows, 11, rows, n_in)
        xt = torch.from_numpy(x).cuda()
        y_load = loaded.forward(xt)
        y_made = made.forward(xt)
        torch.cuda.synchronize()
        y_load = y_load.cpu().numpy()
        assert np.array_equal(y_load.view(np.uint16), y_made.cpu().numpy().view(np.uint16)), rows
        ref = oracle.forward(x, tr, s16, v16, k, cb, bias=b16, mode=1)
        check_linear(y_load, ref, f"loaded k={k} cb={cb} rows={rows}")
    del loaded, made
    ck.close()


def _fixture_shard(golden, tmp_path, name):
    import mlxl3_amd

    fix = json.loads((golden / "real_tiles" / f"{name}.json").read_text())
    nr, nc, nw = fix["shape"]
    rng = np.random.default_rng(sum(map(ord, name)))
    words = rng.integers(0, 1 << 16, size=(nr * nc, nw), dtype=np.uint16)
    for tile in fix["tiles"]:
        words[tile["tile"]] = tile["packed"]
    prefix = fix["tensor"].removesuffix(".trellis")
    tr = words.reshape(nr, nc, nw)
    suh = synth.signs_scales(3, 1, nr * 16)
    svh = synth.signs_scales(3, 2, nc * 16)
    tensors = synth.exl3_tensors(prefix, tr, suh, svh, cb=fix["mode"], signed=fix["dtype"] == "I16")
    root = synth.write_checkpoint(tmp_path / name, [tensors], {prefix: {"quant_format": "exl3"}})
    return fix, prefix, tr, suh, svh, mlxl3_amd.Checkpoint(root)


@pytest.mark.parametrize("name", ["flash", "qwen-dense", "qwen-moe", "lfm-moe"])
def test_real_tile_checkpoint(golden, tmp_path, name):
    """Real tiles through the loader's read path and the GPU decoder, then the
    loaded projection at the real tensor's shape against the oracle."""
    import mlxl3_amd

    torch = torch_mod()
    print(f"real-tile checkpoint {name}", flush=True)
    fix, prefix, tr, suh, svh, ck = _fixture_shard(golden, tmp_path, name)
    k, cb = fix["k"], fix["mode"]
    words = ck.read(fix["tensor"]).view(np.uint16).reshape(-1, 16 * k)
    picked = np.stack([words[t["tile"]] for t in fix["tiles"]])
    states, values = mlxl3_amd.decode_tiles(dev(picked), k, cb)
    torch.cuda.synchronize()
    for i, t in enumerate(fix["tiles"]):
        assert states[i].cpu().numpy().astype(np.uint16).tolist() == t["states"], (name, t["tile"])
        assert values[i].cpu().numpy().view(np.uint16).tolist() == t["f16_bits"], (name, t["tile"])
    lin = mlxl3_amd.Exl3Linear.from_checkpoint(ck, prefix)
    assert (lin.k, lin.cb) == (k, cb)
    n_in = tr.shape[0] * 16
    for rows in (1, 20):
        x = synth.activations(90 + rows, 12, rows, n_in)
        y = lin.forward(torch.from_numpy(x).cuda())
        torch.cuda.synchronize()
        ref = oracle.forward(x, tr, suh, svh, k, cb, mode=1)
        check_linear(y.cpu().numpy(), ref, f"{name} rows={rows}")
    del lin
    ck.close()


def _bank_tensors(prefix, experts, in_f, hidden, k, cb, names, seed=5, replace_gate0=None):
    tensors, layers = {}, []
    for e in range(experts):
        per = []
        for j, (p, (i, o)) in enumerate(zip(names, ((in_f, hidden), (in_f, hidden), (hidden, in_f)))):
            t, suh, svh, _ = synth.linear_layer(seed, 100 + 3 * e + j, i, o, k)
            # keep the SwiGLU glue in range: output scales ~ 1/sqrt(fan-in)
            svh = (svh.astype(np.float32) / np.sqrt(i)).astype(np.float16)
            if e == 0 and j == 0 and replace_gate0 is not None:
                t = replace_gate0
            tensors.update(synth.exl3_tensors(f"{prefix}.{e}.{p}", t, suh, svh, cb=cb))
            per.append((t, suh, svh))
        layers.append(per)
    return tensors, layers


def _numpy_bank(layers):
    """moe.rs:756-800 by numpy: gate trellises then up trellises concatenated on
    the output-tile axis, down trellises likewise, scales stacked per expert."""
    gates = [l[0] for l in layers]
    ups = [l[1] for l in layers]
    downs = [l[2] for l in layers]
    gu = np.concatenate([g[0] for g in gates] + [u[0] for u in ups], axis=1)
    gu_suh = np.stack([np.stack([g[1], u[1]]) for g, u in zip(gates, ups)])
    gu_svh = np.stack([np.stack([g[2], u[2]]) for g, u in zip(gates, ups)])
    dn = np.concatenate([d[0] for d in downs], axis=1)
    return gu, gu_suh, gu_svh, dn, np.stack([d[1] for d in downs]), np.stack([d[2] for d in downs])


def _moe_check(y, ref, label):
    y64, r64 = y.astype(np.float64), ref.astype(np.float64)
    rel = np.linalg.norm(y64 - r64) / np.linalg.norm(r64)
    mx = np.abs(y64 - r64).max() / np.sqrt(np.mean(r64 ** 2))
    print(f"{label}: rel_l2={rel:.3e} max_abs/rms={mx:.3e}", flush=True)
    assert rel <= TOL_REL and mx <= MOE_TOL_RMS, (label, rel, mx)


@pytest.mark.parametrize(
    "names, k, cb, experts, top_k, in_f, hidden, rows",
    [
        (("gate_proj", "up_proj", "down_proj"), 3, 1, 4, 2, 256, 384, 9),
        (("w1", "w3", "w2"), 2, 2, 6, 3, 384, 256, 70),
    ],
)
def test_moe_load_equals_create(tmp_path, names, k, cb, experts, top_k, in_f, hidden, rows):
    import mlxl3_amd

    torch = torch_mod()
    print(f"moe load {names[0]} k={k} cb={cb} E={experts} rows={rows}", flush=True)
    tensors, layers = _bank_tensors("model.layers.2.mlp.experts", experts, in_f, hidden, k, cb, names)
    # the bank's projections are exl3 modules of tensor_storage, as in a real checkpoint
    storage = {n.removesuffix(".trellis"): {"quant_format": "exl3"} for n in tensors if n.endswith(".trellis")}
    half = len(tensors) // 2
    items = list(tensors.items())
    root = synth.write_checkpoint(tmp_path / "m", [dict(items[:half]), dict(items[half:])], storage)
    ck = mlxl3_amd.Checkpoint(root)
    if names[0] == "w1":
        loaded = mlxl3_amd.Exl3SwitchGlu.from_lfm_checkpoint(ck, "model.layers.2.mlp.experts", experts, top_k)
    else:
        loaded = mlxl3_amd.Exl3SwitchGlu.from_checkpoint(ck, "model.layers.2.mlp.experts", experts, top_k)
    assert (loaded.input, loaded.hidden, loaded.k, loaded.cb) == (in_f, hidden, k, cb)
    bank = _numpy_bank(layers)
    made = mlxl3_amd.Exl3SwitchGlu(*[dev(a) for a in bank], top_k=top_k, k=k, cb=cb)
    x = synth.activations(31, 1, rows, in_f)
    sel, sc = synth.moe_routes(31, 2, rows, experts, top_k)
    y_load = loaded.forward(dev(x), dev(sel), dev(sc))
    y_made = made.forward(dev(x), dev(sel), dev(sc))
    torch.cuda.synchronize()
    y_load = y_load.cpu().numpy()
    assert np.array_equal(y_load.view(np.uint16), y_made.cpu().numpy().view(np.uint16))
    _moe_check(y_load, oracle.moe_forward(x, sel, sc, *bank, k, cb), f"moe load {names[0]}")
    del loaded, made
    ck.close()


def test_moe_load_gemma_equals_create_gelu(tmp_path):
    """Exl3SwitchGlu::from_gemma_checkpoint (moe.rs:663-680): the GELU bank loaded
    from a checkpoint equals the one created from the same tensors, bit for bit,
    and both follow the oracle's forward_gelu."""
    import mlxl3_amd

    torch = torch_mod()
    names = ("gate_proj", "up_proj", "down_proj")
    experts, top_k, in_f, hidden, k, cb, rows, logical = 4, 2, 256, 384, 3, 0, 12, 320
    print(f"moe load gemma k={k} E={experts} logical={logical}", flush=True)
    tensors, layers = _bank_tensors("model.layers.1.experts", experts, in_f, hidden, k, cb, names)
    storage = {n.removesuffix(".trellis"): {"quant_format": "exl3"} for n in tensors if n.endswith(".trellis")}
    root = synth.write_checkpoint(tmp_path / "g", [tensors], storage)
    ck = mlxl3_amd.Checkpoint(root)
    loaded = mlxl3_amd.Exl3SwitchGlu.from_gemma_checkpoint(ck, "model.layers.1.experts", experts,
                                                           top_k, logical)
    assert (loaded.activation, loaded.logical_hidden) == ("gelu", logical)
    bank = _numpy_bank(layers)
    made = mlxl3_amd.Exl3SwitchGlu(*[dev(a) for a in bank], top_k=top_k, k=k, cb=cb,
                                   activation="gelu", logical_hidden=logical)
    x = synth.activations(33, 1, rows, in_f)
    sel, sc = synth.moe_routes(33, 2, rows, experts, top_k)
    y_load = loaded.forward(dev(x), dev(sel), dev(sc))
    y_made = made.forward(dev(x), dev(sel), dev(sc))
    torch.cuda.synchronize()
    y_load = y_load.cpu().numpy()
    assert np.array_equal(y_load.view(np.uint16), y_made.cpu().numpy().view(np.uint16))
    _moe_check(y_load, oracle.moe_forward(x, sel, sc, *bank, k, cb, activation="gelu",
                                          logical_hidden=logical), "moe load gemma")
    del loaded, made
    ck.close()


@pytest.mark.parametrize("name, names", [("qwen-moe", ("gate_proj", "up_proj", "down_proj")),
                                         ("lfm-moe", ("w1", "w3", "w2"))])
def test_moe_bank_with_real_expert_tiles(golden, tmp_path, name, names):
    """A 4-expert bank at the real expert shape whose expert-0 gate holds the
    real tiles (qwen-moe: 2048 x 512 K3 MCG; lfm-moe: 2048 x 1536 K4 MCG)."""
    import mlxl3_amd

    torch = torch_mod()
    print(f"moe real-tile bank {name}", flush=True)
    fix = json.loads((golden / "real_tiles" / f"{name}.json").read_text())
    nr, nc, nw = fix["shape"]
    rng = np.random.default_rng(11)
    words = rng.integers(0, 1 << 16, size=(nr * nc, nw), dtype=np.uint16)
    for tile in fix["tiles"]:
        words[tile["tile"]] = tile["packed"]
    prefix = fix["tensor"].removesuffix(".0." + names[0] + ".trellis")
    k, cb, experts, top_k = fix["k"], fix["mode"], 4, 2
    tensors, layers = _bank_tensors(prefix, experts, nr * 16, nc * 16, k, cb, names,
                                    replace_gate0=words.reshape(nr, nc, nw))
    assert fix["tensor"] in tensors
    storage = {n.removesuffix(".trellis"): {"quant_format": "exl3"} for n in tensors if n.endswith(".trellis")}
    root = synth.write_checkpoint(tmp_path / name, [tensors], storage)
    ck = mlxl3_amd.Checkpoint(root)
    moe = mlxl3_amd.Exl3SwitchGlu.from_checkpoint(ck, prefix, experts, top_k, names)
    x = synth.activations(41, 1, 12, nr * 16)
    sel, sc = synth.moe_routes(41, 2, 12, experts, top_k)
    y = moe.forward(dev(x), dev(sel), dev(sc))
    torch.cuda.synchronize()
    _moe_check(y.cpu().numpy(), oracle.moe_forward(x, sel, sc, *_numpy_bank(layers), k, cb),
               f"moe real-tile bank {name}")
    del moe
    ck.close()


# ---- codec ops over banks and checkpoints (main.rs:627-725) ----


def test_codec_mlx_switch_equals_the_api():
    import mlxl3_amd
    from codec_client import run

    torch = torch_mod()
    in_f, hidden, experts, top_k, rows, k, cb = 256, 256, 6, 2, 5, 3, 1
    layer = synth.moe_layer(9, 500, in_f, hidden, experts, k)
    x = synth.activations(9, 510, rows, in_f)
    sel, sc = synth.moe_routes(9, 520, rows, experts, top_k)
    gu, gu_suh, gu_svh, dn, dsu, dsv = layer
    u16 = lambda a: np.ascontiguousarray(a).view(np.uint16).ravel().tolist()
    req = {"op": "mlx-switch", "key_heads": experts, "top_k": top_k, "cols": hidden, "k": k,
           "mode": cb, "selected": sel.ravel().tolist(), "beta": u16(sc), "x": u16(x),
           "data": u16(gu), "down_data": u16(dn), "suh": u16(gu_suh), "svh": u16(gu_svh),
           "down_suh": u16(dsu), "down_svh": u16(dsv)}
    (row,) = run([req])
    got = np.array(row["data"], np.uint16).reshape(rows, in_f)
    moe = mlxl3_amd.Exl3SwitchGlu(*[dev(a) for a in layer], top_k=top_k, k=k, cb=cb)
    y = moe.forward(dev(x), dev(sel), dev(sc))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got, y.cpu().numpy().view(np.uint16))
    _moe_check(got.view(np.float16), oracle.moe_forward(x, sel, sc, *layer, k, cb), "codec mlx-switch")


@pytest.mark.parametrize("model_type, names", [("qwen3_moe", ("gate_proj", "up_proj", "down_proj")),
                                               ("lfm2_moe", ("w1", "w3", "w2"))])
def test_codec_mlx_checkpoint_switch_equals_the_loader(tmp_path, model_type, names):
    import mlxl3_amd
    from codec_client import run

    torch = torch_mod()
    experts, top_k, in_f, hidden, k, cb = 4, 2, 256, 256, 2, 0
    prefix = "model.layers.0.mlp.experts"
    tensors, layers = _bank_tensors(prefix, experts, in_f, hidden, k, cb, names)
    storage = {n.removesuffix(".trellis"): {"quant_format": "exl3"} for n in tensors if n.endswith(".trellis")}
    root = synth.write_checkpoint(tmp_path / model_type, [tensors], storage, model_type=model_type)
    x = synth.activations(41, 1, 1, in_f)
    sel, sc = synth.moe_routes(41, 2, 1, experts, top_k)
    req = {"op": "mlx-checkpoint-switch", "path": str(root), "prefix": prefix,
           "key_heads": experts, "selected": sel.ravel().tolist(),
           "beta": sc.view(np.uint16).ravel().tolist(), "x": x.view(np.uint16).ravel().tolist()}
    (row,) = run([req])
    ck = mlxl3_amd.Checkpoint(root)
    loaded = mlxl3_amd.Exl3SwitchGlu.from_checkpoint(ck, prefix, experts, top_k, names)
    y = loaded.forward(dev(x), dev(sel), dev(sc))
    torch.cuda.synchronize()
    print(f"codec mlx-checkpoint-switch {model_type}: {len(row['data'])} values", flush=True)
    np.testing.assert_array_equal(np.array(row["data"], np.uint16), y.cpu().numpy().view(np.uint16).ravel())
    del loaded
    ck.close()


def test_codec_mlx_checkpoint_group(tmp_path):
    import mlxl3_amd
    from codec_client import run

    torch = torch_mod()
    tensors, want = {}, {}
    specs = {"q": (256, 256, 3), "k": (256, 128, 3), "v": (256, 128, 3), "o": (256, 256, 2)}
    for i, (name, (n_in, n_out, k)) in enumerate(specs.items()):
        t, suh, svh, _ = synth.linear_layer(12, 200 + i, n_in, n_out, k)
        tensors.update(synth.exl3_tensors(f"model.layers.0.attn.{name}_proj", t, suh, svh))
    storage = {n.removesuffix(".trellis"): {"quant_format": "exl3"} for n in tensors if n.endswith(".trellis")}
    root = synth.write_checkpoint(tmp_path / "g", [tensors], storage)
    x = synth.activations(12, 9, 1, 256)
    xs = x.view(np.uint16).ravel().tolist()
    pre = lambda names: [f"model.layers.0.attn.{n}_proj" for n in names]
    rows = run([{"op": "mlx-checkpoint-group", "path": str(root), "prefixes": pre("qkv"), "x": xs},
                {"op": "mlx-checkpoint-group", "path": str(root), "prefixes": pre("qo"), "x": xs},
                {"op": "mlx-checkpoint-group", "path": str(root), "prefixes": [], "x": xs}])
    assert rows[0]["data"]["grouped"] is True and rows[1]["data"]["grouped"] is False
    assert "empty projection bundle" in rows[2]["error"]
    ck = mlxl3_amd.Checkpoint(root)
    for row, names in ((rows[0], "qkv"), (rows[1], "qo")):
        for out, p in zip(row["data"]["outputs"], pre(names)):
            lin = mlxl3_amd.Exl3Linear.from_checkpoint(ck, p)
            y = lin.forward(torch.from_numpy(x).cuda())
            torch.cuda.synchronize()
            np.testing.assert_array_equal(np.array(out, np.uint16), y.cpu().numpy().view(np.uint16).ravel())
            del lin
    ck.close()
