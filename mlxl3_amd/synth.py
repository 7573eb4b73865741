"""Seeded synthetic EXL3 layers and activations (bench and test inputs).

Stream: splitmix64 over a counter keyed by (seed, tensor id), so every tensor
is reproducible on any host and independent of generation order.

* trellis: uniform random u16 words -- every bitstream is a valid trellis,
  since the window read of codec.rs:40-50 is total;
* suh / svh: f16(s * u) with s = +-1 and u = 0.5 + U[0, 1);
* activations: f16(N(0, 1)) by Box-Muller on 53-bit uniforms, optionally with
  a fraction of outlier channels scaled before rounding.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

_GOLD = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def u64_stream(seed: int, tensor_id: int, n: int) -> np.ndarray:
    """n splitmix64 outputs for (seed, tensor_id)."""
    base = _mix(np.array([(seed * 0x100000001B3 + tensor_id) & 0xFFFFFFFFFFFFFFFF], np.uint64))[0]
    with np.errstate(over="ignore"):
        ctr = base + (np.arange(1, n + 1, dtype=np.uint64) * _GOLD)
        return _mix(ctr)


def uniform(seed: int, tensor_id: int, n: int) -> np.ndarray:
    """U[0, 1) from the top 53 bits."""
    return (u64_stream(seed, tensor_id, n) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def trellis(seed: int, tensor_id: int, in_features: int, out_features: int, k: int) -> np.ndarray:
    """[in/16, out/16, 16k] uint16."""
    words = in_features // 16 * (out_features // 16) * 16 * k
    raw = u64_stream(seed, tensor_id, (words + 3) // 4)
    return raw.view(np.uint16)[:words].reshape(in_features // 16, out_features // 16, 16 * k).copy()


def signs_scales(seed: int, tensor_id: int, n: int) -> np.ndarray:
    """f16(+-1 * U(0.5, 1.5)), [n] float16."""
    r = u64_stream(seed, tensor_id, n)
    sign = np.where((r & np.uint64(1)) == 0, 1.0, -1.0)
    u = 0.5 + (r >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))
    return (sign * u).astype(np.float16)


def normal(seed: int, tensor_id: int, n: int) -> np.ndarray:
    """N(0, 1) float64 by Box-Muller."""
    m = (n + 1) // 2
    u1 = uniform(seed, tensor_id, 2 * m).reshape(m, 2)
    r = np.sqrt(-2.0 * np.log1p(-u1[:, 0]))
    t = 2.0 * np.pi * u1[:, 1]
    return np.stack([r * np.cos(t), r * np.sin(t)], axis=1).reshape(-1)[:n]


def activations(seed: int, tensor_id: int, rows: int, features: int, outlier_frac: float = 0.0,
                outlier_scale: float = 20.0) -> np.ndarray:
    """f16 [rows, features] ~ N(0,1); round(outlier_frac*features) channels x outlier_scale."""
    x = normal(seed, tensor_id, rows * features).reshape(rows, features)
    count = int(round(outlier_frac * features))
    if count:
        # partial Fisher-Yates over the channel indices
        idx = np.arange(features)
        r = u64_stream(seed, tensor_id + 7919, count)
        for i in range(count):
            j = i + int(r[i] % np.uint64(features - i))
            idx[i], idx[j] = idx[j], idx[i]
        x[:, idx[:count]] *= outlier_scale
    return x.astype(np.float16)


def linear_layer(seed: int, base_id: int, in_features: int, out_features: int, k: int,
                 bias: bool = False):
    """(trellis, suh, svh, bias) numpy arrays of one synthetic EXL3 linear."""
    t = trellis(seed, base_id, in_features, out_features, k)
    suh = signs_scales(seed, base_id + 1, in_features)
    svh = signs_scales(seed, base_id + 2, out_features)
    b = signs_scales(seed, base_id + 3, out_features) if bias else None
    return t, suh, svh, b


def moe_layer(seed: int, base_id: int, in_features: int, hidden: int, experts: int, k: int):
    """SwitchGLU expert banks in the reference's layout (moe.rs:756-760, 835-870).

    Returns (gu_trellis [in/16, 2*E*H/16, 16k], gu_suh [E, 2, in], gu_svh [E, 2, H],
    down_trellis [H/16, E*in/16, 16k], down_suh [E, H], down_svh [E, in]); gate tiles
    of expert e sit at tile columns [e*H/16, (e+1)*H/16), up tiles at [(E+e)*H/16, ...).
    The output scales carry 1/sqrt(fan-in), as a quantized checkpoint's svh does, so the
    SwiGLU product stays in f16 range: svh = f16(+-U(0.5, 1.5) / sqrt(fan_in)).
    """
    gu = trellis(seed, base_id, in_features, 2 * experts * hidden, k)
    gu_suh = signs_scales(seed, base_id + 1, experts * 2 * in_features).reshape(experts, 2, in_features)
    gu_svh = (signs_scales(seed, base_id + 2, experts * 2 * hidden).astype(np.float64)
              / np.sqrt(in_features)).astype(np.float16).reshape(experts, 2, hidden)
    down = trellis(seed, base_id + 3, hidden, experts * in_features, k)
    down_suh = signs_scales(seed, base_id + 4, experts * hidden).reshape(experts, hidden)
    down_svh = (signs_scales(seed, base_id + 5, experts * in_features).astype(np.float64)
                / np.sqrt(hidden)).astype(np.float16).reshape(experts, in_features)
    return gu, gu_suh, gu_svh, down, down_suh, down_svh


def moe_routes(seed: int, tensor_id: int, rows: int, experts: int, top_k: int,
               dtype=np.float16):
    """Top-k routing from softmax(N(0,1) logits), probabilities renormalised over the top k.

    Returns (selected uint32 [rows, top_k] in descending-probability order,
    scores [rows, top_k] of `dtype`, float16 by default).
    """
    logits = normal(seed, tensor_id, rows * experts).reshape(rows, experts).astype(np.float32)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    order = np.argsort(-p, axis=1, kind="stable")[:, :top_k]
    top = np.take_along_axis(p, order, axis=1)
    top /= top.sum(axis=1, keepdims=True)
    return order.astype(np.uint32), top.astype(dtype)


# ---------------------------------------------------------------------------
# safetensors / checkpoint writers (synthetic EXL3 model directories)
# ---------------------------------------------------------------------------
_ST_DTYPES = {
    np.dtype("bool"): "BOOL", np.dtype("uint8"): "U8", np.dtype("int8"): "I8",
    np.dtype("uint16"): "U16", np.dtype("int16"): "I16", np.dtype("float16"): "F16",
    np.dtype("uint32"): "U32", np.dtype("int32"): "I32", np.dtype("float32"): "F32",
    np.dtype("uint64"): "U64", np.dtype("int64"): "I64", np.dtype("float64"): "F64",
}


def safetensors_bytes(tensors: dict, metadata: dict | None = None, pad_to: int = 8) -> bytes:
    """One safetensors file: 8-byte little-endian header length, JSON header,
    payloads packed in insertion order.  A value is a numpy array or a
    (dtype string, array) pair whose bytes are stored as given (e.g.
    ("BF16", uint16 bits))."""
    header, blobs, offset = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, value in tensors.items():
        dtype, arr = value if isinstance(value, tuple) else (_ST_DTYPES[value.dtype], value)
        arr = np.asarray(arr, order="C")  # keeps 0-d scalars 0-d
        raw = arr.astype(arr.dtype.newbyteorder("<"), copy=False).tobytes()
        header[name] = {"dtype": dtype, "shape": list(arr.shape),
                        "data_offsets": [offset, offset + len(raw)]}
        blobs.append(raw)
        offset += len(raw)
    text = json.dumps(header, separators=(",", ":")).encode()
    text += b" " * (-len(text) % pad_to)
    return len(text).to_bytes(8, "little") + text + b"".join(blobs)


def write_checkpoint(root, shards: list, storage: dict, model_type: str = "llama",
                     bits: float | None = 4.0, index: bool = True, tokenizer: bool = True) -> Path:
    """An EXL3 model directory: config.json, quantization_config.json
    (quant_method "exl3", tensor_storage = storage), tokenizer.json, shards
    model-0000i-of-0000n.safetensors and their weight-map index."""
    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    (root / "config.json").write_text(json.dumps({"model_type": model_type}))
    quant = {"quant_method": "exl3", "tensor_storage": storage}
    if bits is not None:
        quant["bits"] = bits
    (root / "quantization_config.json").write_text(json.dumps(quant))
    if tokenizer:
        (root / "tokenizer.json").write_text("{}")
    weight_map = {}
    n = len(shards)
    for i, tensors in enumerate(shards):
        name = "model.safetensors" if n == 1 else f"model-{i + 1:05d}-of-{n:05d}.safetensors"
        (root / name).write_bytes(safetensors_bytes(tensors))
        weight_map.update({t: name for t in tensors})
    if index:
        (root / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    return root


def exl3_tensors(prefix: str, trellis_u16: np.ndarray, suh: np.ndarray, svh: np.ndarray,
                 bias: np.ndarray | None = None, cb: int = 0, legacy_names: bool = False,
                 scale_dtype: str = "F16", signed: bool = True) -> dict:
    """The tensors of one EXL3 projection as a checkpoint stores them:
    {prefix}.trellis (I16 or U16), .suh/.svh (or legacy .su/.sv) as F16, BF16
    or F32, optional .bias (F16), and a .mcg / .mul1 flag tensor for the MCG /
    MUL1 codebooks."""
    def scale(v):
        v32 = np.asarray(v, dtype=np.float32)
        if scale_dtype == "F32":
            return v32
        if scale_dtype == "BF16":
            bits = v32.view(np.uint32)
            # round to nearest even into bfloat16 bits
            rounded = (bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
            return ("BF16", rounded.astype(np.uint16))
        return v32.astype(np.float16)
    su, sv = ("su", "sv") if legacy_names else ("suh", "svh")
    t = trellis_u16.view(np.int16) if signed else trellis_u16
    out = {f"{prefix}.trellis": t, f"{prefix}.{su}": scale(suh), f"{prefix}.{sv}": scale(svh)}
    if bias is not None:
        out[f"{prefix}.bias"] = np.asarray(bias, dtype=np.float16)
    if cb == 1:
        out[f"{prefix}.mcg"] = np.array(0xCBAC1FED, dtype=np.uint32).view(np.int32).reshape(())
    elif cb == 2:
        out[f"{prefix}.mul1"] = np.array(0x83DCD12D, dtype=np.uint32).view(np.int32).reshape(())
    return out
