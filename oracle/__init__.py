"""ctypes wrapper of the C oracle (oracle/liboracle_exl3.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.  The
product package (mlxl3_amd) never imports it.

Function-by-function citations are in exl3_oracle.h / exl3_oracle.c.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle_exl3.so"

_lib = None
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_vp = ctypes.c_void_p

DT_F16, DT_F32, DT_BF16 = 9, 10, 12


def build() -> Path:
    """Compile the oracle with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-B", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.exl3o_f16_to_f32.restype = ctypes.c_float
        L.exl3o_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.exl3o_f32_to_f16.restype = ctypes.c_uint16
        L.exl3o_f32_to_f16.argtypes = [ctypes.c_float]
        L.exl3o_f64_to_f16.restype = ctypes.c_uint16
        L.exl3o_f64_to_f16.argtypes = [ctypes.c_double]
        L.exl3o_bf16_to_f32.restype = ctypes.c_float
        L.exl3o_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.exl3o_f32_to_bf16.restype = ctypes.c_uint16
        L.exl3o_f32_to_bf16.argtypes = [ctypes.c_float]
        L.exl3o_swiglu.restype = None
        L.exl3o_swiglu.argtypes = [_u16p, _u16p, _u16p, ctypes.c_int64]
        L.exl3o_swiglu_down_input.restype = ctypes.c_int
        L.exl3o_swiglu_down_input.argtypes = [_f32p, _u16p, _u16p, _u32p, ctypes.c_int64,
                                              ctypes.c_int, ctypes.c_int, _u16p]
        L.exl3o_finish_and_reduce.restype = ctypes.c_int
        L.exl3o_finish_and_reduce.argtypes = [_f32p, _u16p, _vp, ctypes.c_int, ctypes.c_int64,
                                              ctypes.c_int, ctypes.c_int, _vp]
        L.exl3o_result_dtype.restype = ctypes.c_int
        L.exl3o_result_dtype.argtypes = [ctypes.c_int, ctypes.c_int]
        L.exl3o_geglu.restype = None
        L.exl3o_geglu.argtypes = [_u16p, _u16p, _u16p, ctypes.c_int64]
        L.exl3o_codeword.restype = ctypes.c_uint16
        L.exl3o_codeword.argtypes = [ctypes.c_uint16, ctypes.c_int]
        L.exl3o_codebook.restype = None
        L.exl3o_codebook.argtypes = [ctypes.c_int, _u16p]
        L.exl3o_unpack.restype = ctypes.c_int
        L.exl3o_unpack.argtypes = [_u16p, ctypes.c_int64, ctypes.c_int, _u16p]
        L.exl3o_pack.restype = ctypes.c_int
        L.exl3o_pack.argtypes = [_u16p, ctypes.c_int64, ctypes.c_int, _u16p]
        L.exl3o_permutation.restype = None
        L.exl3o_permutation.argtypes = [_u16p]
        L.exl3o_reconstruct_inner.restype = ctypes.c_int
        L.exl3o_reconstruct_inner.argtypes = [_u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
                                              ctypes.c_int64, _u16p]
        L.exl3o_h128_f32.restype = None
        L.exl3o_h128_f32.argtypes = [_f32p, ctypes.c_int64]
        L.exl3o_h128_staged.restype = None
        L.exl3o_h128_staged.argtypes = [_f32p, ctypes.c_int64]
        L.exl3o_forward.restype = ctypes.c_int
        L.exl3o_forward.argtypes = [ctypes.c_int, _vp, ctypes.c_int, ctypes.c_int64, _u16p,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _u16p,
                                    _u16p, _vp, _vp, _vp, ctypes.c_int]
        L.exl3o_prologue.restype = ctypes.c_int
        L.exl3o_prologue.argtypes = [_vp, ctypes.c_int, ctypes.c_int64, ctypes.c_int, _u16p, _u16p]
        L.exl3o_moe_forward.restype = ctypes.c_int
        L.exl3o_moe_forward.argtypes = [_vp, ctypes.c_int, ctypes.c_int64, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, _u16p, _u16p, _u16p, _u16p, _u16p, _u16p,
                                        _u32p, _vp, ctypes.c_int, _vp, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int]
        L.exl3o_expert_mapped.restype = ctypes.c_int
        L.exl3o_expert_mapped.argtypes = [_vp, ctypes.c_int, ctypes.c_int64, ctypes.c_int, _u16p,
                                          _u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _u32p,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          _vp, ctypes.c_int, _vp, ctypes.c_int]
        _lib = L
    return _lib


def _u16(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    if a.dtype == np.int16:
        a = a.view(np.uint16)
    return np.ascontiguousarray(a, dtype=np.uint16)


def _dtype_code(a: np.ndarray, dtype=None) -> int:
    """Dtype code of an activation array: float16, float32, or (dtype="bf16")
    bfloat16 bits held in a uint16 array (numpy has no bfloat16)."""
    if dtype == "bf16":
        if a.dtype != np.uint16:
            raise ValueError("bf16 arrays are passed as their uint16 bits")
        return DT_BF16
    if a.dtype == np.float16:
        return DT_F16
    if a.dtype == np.float32:
        return DT_F32
    raise ValueError(f"oracle activations are float16, float32 or bf16 bits, got {a.dtype}")


_NP_OF_CODE = {DT_F16: np.float16, DT_F32: np.float32, DT_BF16: np.uint16}


def result_dtype(x_code: int, has_bias: bool) -> int:
    """exl3o_result_dtype: the projection's output dtype code."""
    return int(lib().exl3o_result_dtype(int(x_code), int(bool(has_bias))))


def codeword(state: int, cb: int) -> int:
    return int(lib().exl3o_codeword(state & 0xFFFF, cb))


def codebook(cb: int) -> np.ndarray:
    """f16 bits of every state, [65536] uint16."""
    out = np.empty(65536, np.uint16)
    lib().exl3o_codebook(cb, out)
    return out


def unpack(packed, k: int) -> np.ndarray:
    p = _u16(packed).ravel()
    if p.size % (16 * k):
        raise ValueError("packed length is not a whole tile")
    tiles = p.size // (16 * k)
    out = np.empty(tiles * 256, np.uint16)
    if lib().exl3o_unpack(p, tiles, k, out):
        raise ValueError(f"K must be in 1..=8, got {k}")
    return out.reshape(tiles, 256)


def pack(states, k: int) -> np.ndarray:
    s = _u16(states).ravel()
    if s.size % 256:
        raise ValueError("encoded length must be a multiple of 256")
    tiles = s.size // 256
    out = np.empty(tiles * 16 * k, np.uint16)
    if lib().exl3o_pack(s, tiles, k, out):
        raise ValueError(f"K must be in 1..=8, got {k}")
    return out.reshape(tiles, 16 * k)


def permutation() -> np.ndarray:
    out = np.empty(256, np.uint16)
    lib().exl3o_permutation(out)
    return out.astype(np.int64)


def reconstruct_inner(packed, k: int, cb: int, rows: int, cols: int) -> np.ndarray:
    """Dense W_inner [rows, cols] float16 (codec.rs:158-190)."""
    out = np.empty(rows * cols, np.uint16)
    if lib().exl3o_reconstruct_inner(_u16(packed).ravel(), k, cb, rows, cols, out):
        raise ValueError("invalid reconstruct arguments")
    return out.view(np.float16).reshape(rows, cols)


def h128_f32(v) -> np.ndarray:
    a = np.ascontiguousarray(v, dtype=np.float32).copy()
    lib().exl3o_h128_f32(a.reshape(-1), a.size)
    return a


def h128_staged(v) -> np.ndarray:
    a = np.ascontiguousarray(v, dtype=np.float32).copy()
    lib().exl3o_h128_staged(a.reshape(-1), a.size)
    return a


def prologue(x, suh) -> np.ndarray:
    x = np.ascontiguousarray(x)
    rows, n = x.reshape(-1, x.shape[-1]).shape
    out = np.empty(rows * n, np.uint16)
    rc = lib().exl3o_prologue(x.ctypes.data, _dtype_code(x), rows, n, _u16(suh), out)
    if rc:
        raise ValueError("invalid prologue arguments")
    return out.view(np.float16).reshape(rows, n)


def forward(x, trellis, suh, svh, k: int, cb: int, bias=None, mode: int = 1, threads: int = 0,
            return_yhat: bool = False, x_dtype=None):
    """EXL3 linear on the CPU.  mode 1: engine glue semantics; mode 0: ref/forward.py.
    x: float16, float32, or bf16 bits (uint16) with x_dtype="bf16".  The result
    has the projection's output dtype (result_dtype): x's dtype, or float32 for
    bf16 activations with a bias; bf16 results are returned as uint16 bits."""
    x = np.ascontiguousarray(x)
    code = _dtype_code(x, x_dtype)
    n_in = int(x.shape[-1])
    rows = x.size // n_in
    tr = _u16(trellis)
    n_out = int(tr.shape[1]) * 16 if tr.ndim == 3 else int(len(svh))
    y = np.empty((rows, n_out), _NP_OF_CODE[result_dtype(code, bias is not None)])
    yhat = np.empty((rows, n_out), np.float32) if return_yhat else None
    b = None if bias is None else _u16(bias)
    rc = lib().exl3o_forward(mode, x.ctypes.data, code, rows, tr.ravel(), n_in, n_out,
                             k, cb, _u16(suh), _u16(svh), None if b is None else b.ctypes.data,
                             y.ctypes.data, None if yhat is None else yhat.ctypes.data, threads)
    if rc:
        raise ValueError(f"oracle forward failed ({rc})")
    y = y.reshape(*x.shape[:-1], n_out)
    return (y, yhat) if return_yhat else y


def moe_forward(x, selected, scores, gu_trellis, gu_suh, gu_svh, down_trellis, down_suh,
                down_svh, k: int, cb: int, threads: int = 0, activation: str = "silu",
                logical_hidden=None, x_dtype=None, scores_dtype=None) -> np.ndarray:
    """Exl3SwitchGlu::forward (moe.rs:905-975) for activation "silu", and
    forward_gelu (moe.rs:1087-1153) for "gelu" with GEGLU outputs from column
    logical_hidden on set to zero (None: the whole hidden width).  x and
    scores: float16, float32, or bf16 bits (uint16) with x_dtype / scores_dtype
    "bf16".  Returns float16 for f16 scores, float32 otherwise."""
    x = np.ascontiguousarray(x)
    xcode = _dtype_code(x, x_dtype)
    sc = np.ascontiguousarray(scores)
    scode = _dtype_code(sc, scores_dtype)
    rows, n_in = x.shape
    experts, hidden = gu_svh.shape[0], gu_svh.shape[-1]
    top_k = selected.shape[1]
    if activation not in ("silu", "gelu"):
        raise ValueError(f"unknown GLU activation {activation!r}")
    gelu = activation == "gelu"
    logical = hidden if logical_hidden is None else int(logical_hidden)
    y = np.empty((rows, n_in), np.float16 if scode == DT_F16 else np.float32)
    rc = lib().exl3o_moe_forward(x.ctypes.data, xcode, rows, n_in, hidden, experts, top_k, k, cb,
                                 _u16(gu_trellis).ravel(), _u16(gu_suh).ravel(),
                                 _u16(gu_svh).ravel(), _u16(down_trellis).ravel(),
                                 _u16(down_suh).ravel(), _u16(down_svh).ravel(),
                                 np.ascontiguousarray(selected, np.uint32).ravel(),
                                 sc.ctypes.data, scode, y.ctypes.data, int(gelu), logical, threads)
    if rc:
        raise ValueError(f"oracle MoE forward failed ({rc})")
    return y


def expert_mapped(x, suh, trellis, selected, projections: int, out: int, stride_tiles: int,
                  k: int, cb: int, svh=None, raw: bool = False, x_dtype=None,
                  threads: int = 0) -> np.ndarray:
    """expert_mapped (linear.rs:2817-2852) over a route-major bank trellis
    [in/16][bank_tiles][16k]: x [rows][in] (float16, float32, or bf16 bits with
    x_dtype="bf16"), suh [rows][in], selected [routes], rows = routes *
    projections.  raw: float32 [rows][out]; else [rows][out] of x's dtype
    (bf16 as uint16 bits) with svh [rows][out]."""
    x = np.ascontiguousarray(x)
    code = _dtype_code(x, x_dtype)
    rows, n_in = x.shape
    tr = _u16(trellis)
    sel = np.ascontiguousarray(selected, np.uint32).ravel()
    if raw:
        y = np.empty((rows, out), np.float32)
    else:
        y = np.empty((rows, out), _NP_OF_CODE[code])
    sv = None if svh is None else np.ascontiguousarray(_u16(svh)).ravel()
    rc = lib().exl3o_expert_mapped(x.ctypes.data, code, rows, n_in, _u16(suh).ravel(), tr.ravel(),
                                   int(tr.shape[1]), k, cb, sel, int(sel.size), int(projections),
                                   int(out), int(stride_tiles),
                                   None if sv is None else sv.ctypes.data, int(bool(raw)),
                                   y.ctypes.data, threads)
    if rc:
        raise ValueError(f"oracle expert_mapped failed ({rc})")
    return y


def swiglu(gate, up) -> np.ndarray:
    """Array::swiglu (mlx_bridge.cpp:745-749) on f16 arrays of one shape."""
    g = np.ascontiguousarray(np.asarray(gate, dtype=np.float16)).view(np.uint16)
    u = np.ascontiguousarray(np.asarray(up, dtype=np.float16)).view(np.uint16)
    assert g.shape == u.shape
    out = np.empty_like(g)
    lib().exl3o_swiglu(g.reshape(-1), u.reshape(-1), out.reshape(-1), g.size)
    return out.view(np.float16)


def swiglu_down_input(gate_up, gu_svh, down_suh, selected) -> np.ndarray:
    """swiglu_down_input (moe.rs:569-583): f32 [slots*2, hidden] -> f16 [slots, hidden]."""
    gu = np.ascontiguousarray(gate_up, np.float32)
    hidden = gu.shape[-1]
    sel = np.ascontiguousarray(selected, np.uint32).ravel()
    out = np.empty((sel.size, hidden), np.uint16)
    rc = lib().exl3o_swiglu_down_input(gu.ravel(), _u16(gu_svh).ravel(), _u16(down_suh).ravel(),
                                       sel, sel.size, hidden, np.asarray(gu_svh).shape[0],
                                       out.ravel())
    if rc:
        raise ValueError(f"oracle swiglu_down_input failed ({rc})")
    return out.view(np.float16)


def finish_and_reduce(raw, svh, scores, scores_dtype=None) -> np.ndarray:
    """finish_and_reduce (moe.rs:586-609): raw f32 [rows*top_k, width], svh f16
    of the same shape, scores [rows, top_k] (float16, float32, or bf16 bits with
    scores_dtype="bf16") -> [rows, width], float16 for f16 scores, float32
    otherwise."""
    raw = np.ascontiguousarray(raw, np.float32)
    sc = np.ascontiguousarray(scores)
    code = _dtype_code(sc, scores_dtype)
    rows, top_k = sc.shape
    width = raw.shape[-1]
    y = np.empty((rows, width), np.float16 if code == DT_F16 else np.float32)
    rc = lib().exl3o_finish_and_reduce(raw.ravel(), _u16(svh).ravel(), sc.ctypes.data, code, rows,
                                       top_k, width, y.ctypes.data)
    if rc:
        raise ValueError(f"oracle finish_and_reduce failed ({rc})")
    return y


def geglu(gate, up) -> np.ndarray:
    """Array::geglu (mlx_bridge.cpp:764-774) on f16 arrays of one shape."""
    g = np.ascontiguousarray(np.asarray(gate, dtype=np.float16)).view(np.uint16)
    u = np.ascontiguousarray(np.asarray(up, dtype=np.float16)).view(np.uint16)
    assert g.shape == u.shape
    out = np.empty_like(g)
    lib().exl3o_geglu(g.reshape(-1), u.reshape(-1), out.reshape(-1), g.size)
    return out.view(np.float16)


def mlp_forward(x, gate, up, down, mode: int = 1) -> np.ndarray:
    """Dense SwiGLU MLP of a decoder layer (qwen35.rs:303-307): gate and up
    projections of x (f16 outputs), swiglu, down projection.  gate/up/down:
    (trellis, suh, svh, bias, k, cb) tuples."""
    g = forward(x, *gate[:3], gate[4], gate[5], bias=gate[3], mode=mode)
    u = forward(x, *up[:3], up[4], up[5], bias=up[3], mode=mode)
    act = swiglu(g, u)
    return forward(act, *down[:3], down[4], down[5], bias=down[3], mode=mode)
