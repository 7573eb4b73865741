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
