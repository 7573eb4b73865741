"""MI355X (gfx950) EXL3 quantized-linear library: Python mirror of the operator API.

The compute lives in ``libexl3_hip.so`` (hand-written HIP kernels behind the C
ABI of ``include/exl3_hip.h``).  This module mirrors the reference engine's
operator types on top of that ABI, with the same argument meaning and error
behaviour:

* :class:`Exl3Linear`   -- ``Exl3Linear::new`` / ``forward`` (native/src/linear.rs:577-998)
* :class:`Exl3Group`    -- ``Exl3Group::forward`` (linear.rs:2285-2382), one launch
* :func:`swiglu`, :class:`Exl3Mlp` -- ``Array::swiglu`` (mlx_bridge.cpp:745-749) and the
  dense SwiGLU MLP (qwen35.rs:303-307) with the SwiGLU fused into the gate/up epilogue
* :class:`Exl3SwitchGlu` -- ``Exl3SwitchGlu::new`` / ``forward`` (native/src/moe.rs:809-975)
* :func:`decode_tiles`  -- the ``metal-decode`` codec op (exl3.metal:102-109)
* :class:`Checkpoint`   -- ``checkpoint::inspect`` / ``TensorInfo`` (native/src/checkpoint.rs),
  with ``Exl3Linear.from_checkpoint`` and ``Exl3SwitchGlu.from_checkpoint``

PyTorch is used only to own device memory and to name the current stream.
There is no CPU fallback: without the built library every entry point raises.
"""

from __future__ import annotations

import ctypes
import enum
import os
from pathlib import Path
from typing import Optional, Sequence

# EXL3_LIB selects another build of the same ABI (e.g. the sanitizer build of
# the host code, mlxl3_amd/sanitize.py).
LIB_PATH = Path(os.environ.get("EXL3_LIB") or Path(__file__).resolve().parent / "libexl3_hip.so")

__all__ = [
    "codewords",
    "qmv_inner",
    "Exl3Mlp",
    "swiglu",
    "Checkpoint",
    "TensorInfo",
    "Codebook",
    "Exl3Error",
    "Exl3Linear",
    "Exl3Group",
    "Exl3SwitchGlu",
    "decode_tiles",
    "load_library",
    "LIB_PATH",
]


class Codebook(enum.IntEnum):
    """codec.rs:5-23."""

    DEFAULT = 0  # 3INST
    MCG = 1
    MUL1 = 2


class Exl3Error(RuntimeError):
    """A non-zero status from the C ABI, carrying exl3_last_error()."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


_DTYPE_CODES = {}  # torch dtype -> mlx_bridge dtype code, filled lazily
_lib: Optional[ctypes.CDLL] = None

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t

_SIGNATURES = {
    "exl3_last_error": (ctypes.c_char_p, []),
    "exl3_version": (ctypes.c_char_p, []),
    "exl3_linear_create": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, ctypes.POINTER(_vp)]),
    "exl3_linear_destroy": (None, [_vp]),
    "exl3_linear_in_features": (_i32, [_vp]),
    "exl3_linear_out_features": (_i32, [_vp]),
    "exl3_linear_workspace_bytes": (_sz, [_vp, _i64]),
    "exl3_workspace_init": (_i32, [_vp, _sz, _vp]),
    "exl3_linear_output_dtype": (_i32, [_vp, _i32]),
    "exl3_linear_forward": (_i32, [_vp, _vp, _i32, _i64, _vp, _i32, _vp, _sz, _vp]),
    "exl3_linear_noalloc_max_bytes": (_sz, []),
    "exl3_linear_forward_noalloc": (_i32, [_vp, _vp, _i32, _i64, _vp, _i32, _vp]),
    "exl3_group_workspace_bytes": (_sz, [_vp, _i32, _i64]),
    "exl3_group_forward": (_i32, [_vp, _i32, _vp, _i32, _i64, _vp, _vp, _sz, _vp]),
    "exl3_swiglu": (_i32, [_vp, _vp, _vp, _i64, _vp]),
    "exl3_geglu": (_i32, [_vp, _vp, _vp, _i64, _vp]),
    "exl3_mlp_workspace_bytes": (_sz, [_vp, _vp, _vp, _i64]),
    "exl3_mlp_forward": (_i32, [_vp, _vp, _vp, _vp, _i64, _vp, _vp, _sz, _vp]),
    "exl3_moe_create": (
        _i32,
        [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_vp)],
    ),
    "exl3_moe_create_gelu": (
        _i32,
        [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
         ctypes.POINTER(_vp)],
    ),
    "exl3_moe_destroy": (None, [_vp]),
    "exl3_moe_in_features": (_i32, [_vp]),
    "exl3_moe_hidden_features": (_i32, [_vp]),
    "exl3_moe_workspace_bytes": (_sz, [_vp, _i64]),
    "exl3_moe_forward": (_i32, [_vp, _vp, _i32, _i64, _vp, _vp, _i32, _vp, _vp, _sz, _vp]),
    "exl3_swiglu_down_input": (_i32, [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _vp, _vp]),
    "exl3_finish_and_reduce": (_i32, [_vp, _vp, _vp, _i32, _i64, _i32, _i32, _vp, _vp]),
    "exl3_prepare128": (_i32, [_vp, _i64, _i32, _vp, _i64, _vp, _vp]),
    "exl3_debug_fail_launch": (None, [ctypes.c_char_p]),
    "exl3_expert_mapped_workspace_bytes": (_sz, [_i32, _i32, _i64]),
    "exl3_expert_mapped": (
        _i32,
        [_vp, _i32, _i32, _i32, _i32, _vp, _i32, _i64, _vp, _vp, _i32, _i32, _i32, _i32, _vp,
         _i32, _vp, _vp, _sz, _vp],
    ),
    "exl3_decode_tiles": (_i32, [_vp, _i64, _i32, _i32, _vp, _vp, _vp]),
    "exl3_codewords": (_i32, [_vp, _i64, _i32, _vp, _vp]),
    "exl3_pack_tiles": (_i32, [_vp, _i64, _i32, _vp, _vp]),
    "exl3_qmv_inner_workspace_bytes": (_sz, [_i32, _i32]),
    "exl3_qmv_inner": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _sz, _vp]),
    "exl3_checkpoint_open": (_i32, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "exl3_checkpoint_close": (None, [_vp]),
    "exl3_checkpoint_path": (ctypes.c_char_p, [_vp]),
    "exl3_checkpoint_model_type": (ctypes.c_char_p, [_vp]),
    "exl3_checkpoint_bits": (ctypes.c_double, [_vp]),
    "exl3_checkpoint_size_bytes": (ctypes.c_uint64, [_vp]),
    "exl3_checkpoint_module_count": (_i32, [_vp]),
    "exl3_checkpoint_module": (ctypes.c_char_p, [_vp, _i32]),
    "exl3_checkpoint_tensor_count": (_i64, [_vp]),
    "exl3_checkpoint_tensor_name": (ctypes.c_char_p, [_vp, _i64]),
    "exl3_checkpoint_tensor": (_i32, [_vp, ctypes.c_char_p, _vp]),
    "exl3_checkpoint_read": (_i32, [_vp, ctypes.c_char_p, _vp, _sz]),
    "exl3_checkpoint_read_f16": (_i32, [_vp, ctypes.c_char_p, _vp, _sz]),
    "exl3_linear_load": (_i32, [_vp, ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "exl3_moe_load": (
        _i32,
        [_vp, ctypes.c_char_p, _i32, _i32, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p,
         ctypes.POINTER(_vp)],
    ),
    "exl3_moe_load_gemma": (
        _i32, [_vp, ctypes.c_char_p, _i32, _i32, _i32, ctypes.POINTER(_vp)],
    ),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def load_library(path: Optional[Path] = None) -> ctypes.CDLL:
    """Load libexl3_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise Exl3Error(
            -4, f"{p} is missing: build it with `python -m mlxl3_amd.build` (no CPU fallback exists)"
        )
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def _check(status: int) -> None:
    if status != 0:
        msg = load_library().exl3_last_error().decode("utf-8", "replace")
        raise Exl3Error(status, msg)


def _torch():
    import torch

    return torch


def _dtype_code(dtype) -> int:
    torch = _torch()
    if not _DTYPE_CODES:
        _DTYPE_CODES.update({torch.float16: 9, torch.float32: 10, torch.bfloat16: 12})
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise Exl3Error(-1, f"unsupported activation dtype {dtype}") from None


def _code_dtype(code: int):
    _dtype_code(_torch().float16)  # fills the table
    for dtype, c in _DTYPE_CODES.items():
        if c == code:
            return dtype
    raise Exl3Error(-1, f"unsupported dtype code {code}")


def result_dtype(x_dtype, has_bias: bool):
    """Output dtype of a projection (linear.rs:992-995): y.astype(x.dtype) + an
    f16 bias under MLX's promotion -- x's dtype without a bias; with one,
    float16 stays float16 and bfloat16 or float32 give float32."""
    torch = _torch()
    return torch.float32 if has_bias and x_dtype == torch.bfloat16 else x_dtype


def scores_result_dtype(scores_dtype):
    """Output dtype of the SwitchGLU's weighted top-k sum (finish_and_reduce,
    moe.rs:602-608): f16 expert outputs times the scores -- float16 for
    float16 scores, float32 for float32 or bfloat16 ones (MLX promotes)."""
    torch = _torch()
    return torch.float16 if scores_dtype == torch.float16 else torch.float32


def _stream_ptr(device) -> int:
    torch = _torch()
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _require_device(t, name: str, dtypes=None):
    torch = _torch()
    if t is None:
        return None
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise Exl3Error(-1, f"{name} must be a device tensor")
    if dtypes is not None and t.dtype not in dtypes:
        raise Exl3Error(-1, f"{name} has dtype {t.dtype}, expected one of {dtypes}")
    return t.contiguous()


class _Workspace:
    """Per-device zero-initialised workspace, grown on demand.

    A workspace handed to a forward call by its caller must likewise have been
    zero-filled once (``torch.zeros``, or ``exl3_workspace_init``): the split-K
    kernels count arrivals in its first 64 KiB, which every call leaves at zero
    again.  Calls sharing one workspace must not run concurrently (one stream)."""

    def __init__(self):
        self.buf = None

    def get(self, nbytes: int, device):
        torch = _torch()
        nbytes = max(256, (nbytes + 255) // 256 * 256)
        if self.buf is None or self.buf.numel() < nbytes or self.buf.device != device:
            self.buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        return self.buf


class _TensorInfoC(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_char * 8),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * 8),
        ("offset", ctypes.c_uint64),
        ("bytes", ctypes.c_uint64),
        ("shard", ctypes.c_char_p),
    ]


class TensorInfo:
    """TensorInfo (native/src/checkpoint.rs:15-26): dtype, shape, shard file and
    the absolute byte range of the payload in it."""

    __slots__ = ("name", "dtype", "shape", "shard", "offset", "nbytes")

    def __init__(self, name, dtype, shape, shard, offset, nbytes):
        self.name, self.dtype, self.shape = name, dtype, shape
        self.shard, self.offset, self.nbytes = shard, offset, nbytes

    def __repr__(self):
        return f"TensorInfo({self.name!r}, {self.dtype}, {list(self.shape)}, {self.shard!r}@{self.offset})"


# safetensors dtype -> numpy dtype string for Checkpoint.read
_NP_DTYPES = {
    "BOOL": "?", "U8": "u1", "I8": "i1", "F8_E4M3": "u1", "F8_E5M2": "u1", "U16": "<u2",
    "I16": "<i2", "F16": "<f2", "BF16": "<u2", "U32": "<u4", "I32": "<i4", "F32": "<f4",
    "U64": "<u8", "I64": "<i8", "F64": "<f8",
}


class Checkpoint:
    """An inspected EXL3 model directory (``checkpoint::inspect``,
    native/src/checkpoint.rs:197-330): headers validated, no payload read.

    ``modules`` lists the exl3 projection prefixes; ``tensors`` maps every
    tensor name to its :class:`TensorInfo`; :meth:`read` returns one payload
    as a numpy array (BF16 as its raw uint16 bits).
    """

    def __init__(self, path):
        lib = load_library()
        h = _vp()
        _check(lib.exl3_checkpoint_open(str(path).encode(), ctypes.byref(h)))
        self._handle = h
        self.path = lib.exl3_checkpoint_path(h).decode()
        self.model_type = lib.exl3_checkpoint_model_type(h).decode()
        bits = lib.exl3_checkpoint_bits(h)
        self.bits = None if bits != bits else float(bits)
        self.size_bytes = int(lib.exl3_checkpoint_size_bytes(h))
        self.modules = [lib.exl3_checkpoint_module(h, i).decode()
                        for i in range(lib.exl3_checkpoint_module_count(h))]
        self._names = [lib.exl3_checkpoint_tensor_name(h, i).decode()
                       for i in range(lib.exl3_checkpoint_tensor_count(h))]
        self._infos = {}

    @property
    def handle(self):
        return self._handle

    def close(self):
        h = getattr(self, "_handle", None)
        if h is not None and h.value and _lib is not None:
            _lib.exl3_checkpoint_close(h)
        self._handle = None

    __del__ = close

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __contains__(self, name) -> bool:
        return self.info(name, missing_ok=True) is not None

    @property
    def tensor_names(self):
        return list(self._names)

    def info(self, name: str, missing_ok: bool = False) -> Optional[TensorInfo]:
        if name in self._infos:
            return self._infos[name]
        rec = _TensorInfoC()
        status = load_library().exl3_checkpoint_tensor(self._handle, name.encode(), ctypes.byref(rec))
        if status != 0:
            if missing_ok and status == -1:
                return None
            _check(status)
        info = TensorInfo(name, rec.dtype.decode(), tuple(rec.shape[: rec.ndim]), rec.shard.decode(),
                          int(rec.offset), int(rec.bytes))
        self._infos[name] = info
        return info

    def read(self, name: str):
        """TensorInfo::read_bytes (checkpoint.rs:113-125) as a numpy array."""
        import numpy as np

        info = self.info(name)
        out = np.empty(info.nbytes, dtype=np.uint8)
        _check(load_library().exl3_checkpoint_read(self._handle, name.encode(),
                                                   out.ctypes.data_as(_vp), info.nbytes))
        return out.view(np.dtype(_NP_DTYPES[info.dtype])).reshape(info.shape)

    def read_f16(self, name: str):
        """A float tensor rounded to f16 (astype(Float16)) as a numpy float16 array."""
        import numpy as np

        info = self.info(name)
        count = int(np.prod(info.shape, dtype=np.int64))
        out = np.empty(count, dtype=np.float16)
        _check(load_library().exl3_checkpoint_read_f16(self._handle, name.encode(),
                                                       out.ctypes.data_as(_vp), count))
        return out.reshape(info.shape)


class Exl3Linear:
    """Exl3Linear (native/src/linear.rs:424-998) on one MI355X.

    trellis: int16/uint16 tensor [in/16, out/16, 16*k]; suh [in]; svh [out];
    bias [out] or None (any float dtype, stored as f16); k in 1..8; cb a Codebook.
    """

    def __init__(self, trellis, suh, svh, bias=None, k: int = 4, cb: int = Codebook.DEFAULT):
        torch = _torch()
        lib = load_library()
        if not (1 <= int(k) <= 8):
            raise Exl3Error(-1, f"K must be in 1..=8, got {k}")
        shape = tuple(trellis.shape)
        if len(shape) != 3 or shape[2] != 16 * int(k) or any(d <= 0 for d in shape):
            raise Exl3Error(-1, "invalid trellis shape")
        if trellis.dtype not in (torch.int16, torch.uint16):
            raise Exl3Error(-1, "EXL3 trellis must contain 16-bit integers")
        rows, cols = shape[0] * 16, shape[1] * 16
        if rows % 128 or cols % 128:
            raise Exl3Error(-1, "public EXL3 projections require 128-aligned dimensions")
        if tuple(suh.shape) != (rows,) or tuple(svh.shape) != (cols,):
            raise Exl3Error(-1, "EXL3 scales have wrong dimensions")
        if bias is not None and tuple(bias.shape) != (cols,):
            raise Exl3Error(-1, "EXL3 bias has wrong dimensions")
        self.trellis = _require_device(trellis, "trellis")
        self.suh = _require_device(suh, "suh").to(torch.float16).contiguous()
        self.svh = _require_device(svh, "svh").to(torch.float16).contiguous()
        self.bias = None if bias is None else _require_device(bias, "bias").to(torch.float16).contiguous()
        self.k, self.cb = int(k), int(cb)
        self.in_features, self.out_features = rows, cols
        h = _vp()
        _check(
            lib.exl3_linear_create(
                _ptr(self.trellis), rows, cols, self.k, self.cb, _ptr(self.suh), _ptr(self.svh),
                _ptr(self.bias), ctypes.byref(h),
            )
        )
        self._handle = h
        self._ws = _Workspace()

    @classmethod
    def from_checkpoint(cls, checkpoint: "Checkpoint", prefix: str, device=None) -> "Exl3Linear":
        """Exl3Linear::from_checkpoint (linear.rs:454-575): loads {prefix}.trellis,
        suh/su, svh/sv and an optional bias to `device` (default: the current one);
        the codebook follows the {prefix}.mul1 / .mcg flags."""
        torch = _torch()
        device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        h = _vp()
        with torch.cuda.device(device):
            _check(load_library().exl3_linear_load(checkpoint.handle, prefix.encode(), ctypes.byref(h)))
        self = cls.__new__(cls)
        self._handle = h
        self._ws = _Workspace()
        self.trellis = self.suh = self.svh = self.bias = None  # owned by the handle
        lib = load_library()
        self.in_features = int(lib.exl3_linear_in_features(h))
        self.out_features = int(lib.exl3_linear_out_features(h))
        self.k = checkpoint.info(prefix + ".trellis").shape[-1] // 16
        self.cb = (Codebook.MUL1 if prefix + ".mul1" in checkpoint
                   else Codebook.MCG if prefix + ".mcg" in checkpoint else Codebook.DEFAULT)
        self.device = device
        return self

    def __del__(self):
        h = getattr(self, "_handle", None)
        if h is not None and h.value and _lib is not None:
            _lib.exl3_linear_destroy(h)
            self._handle = None

    @property
    def handle(self):
        return self._handle

    def workspace_bytes(self, rows: int) -> int:
        return int(load_library().exl3_linear_workspace_bytes(self._handle, int(rows)))

    @property
    def has_bias(self) -> bool:
        lib = load_library()
        return lib.exl3_linear_output_dtype(self._handle, 12) == 10  # bf16 -> f32 iff a bias

    def output_dtype(self, x_dtype):
        """The dtype forward returns for x_dtype activations (result_dtype)."""
        code = load_library().exl3_linear_output_dtype(self._handle, _dtype_code(x_dtype))
        return _code_dtype(code)

    def forward(self, x, workspace=None):
        """y = linear(x) for x [..., in] (f16, bf16 or f32); y has x's dtype, or
        float32 for bfloat16 activations with a bias (result_dtype).  A given
        workspace must have been zero-filled once (see _Workspace)."""
        torch = _torch()
        x = _require_device(x, "x", (torch.float16, torch.bfloat16, torch.float32))
        if x.shape[-1] != self.in_features or x.numel() % self.in_features:
            raise Exl3Error(-1, f"invalid EXL3 linear input for {self.in_features} inputs")
        rows = x.numel() // self.in_features
        if rows == 0:
            raise Exl3Error(-1, "EXL3 linear input cannot be empty")
        out_dtype = self.output_dtype(x.dtype)
        y = torch.empty(*x.shape[:-1], self.out_features, dtype=out_dtype, device=x.device)
        need = self.workspace_bytes(rows)
        ws = workspace if workspace is not None else self._ws.get(need, x.device)
        _check(
            load_library().exl3_linear_forward(
                self._handle, _ptr(x), _dtype_code(x.dtype), rows, _ptr(y), _dtype_code(out_dtype),
                _ptr(ws), ws.numel() * ws.element_size(), _stream_ptr(x.device),
            )
        )
        return y

    __call__ = forward


class Exl3Group:
    """Exl3Group (linear.rs:2285-2815): up to 8 projections sharing x (same input
    width, K and codebook), one output each, computed in one launch (rows <= 16)
    or one prologue + one QMM launch."""

    def __init__(self, linears: Sequence[Exl3Linear]):
        if not linears:
            raise Exl3Error(-1, "empty EXL3 group")
        first = linears[0]
        for lin in linears:
            if (lin.in_features, lin.k, lin.cb) != (first.in_features, first.k, first.cb):
                raise Exl3Error(-1, "EXL3 group members need the same input width, K and codebook")
        self.linears = list(linears)
        self._handles = (_vp * len(self.linears))(*[l.handle.value for l in self.linears])
        self._ws = _Workspace()

    def workspace_bytes(self, rows: int) -> int:
        return int(load_library().exl3_group_workspace_bytes(self._handles, len(self.linears), int(rows)))

    def forward(self, x):
        torch = _torch()
        x = _require_device(x, "x", (torch.float16, torch.bfloat16, torch.float32))
        n_in = self.linears[0].in_features
        if x.shape[-1] != n_in or x.numel() % n_in:
            raise Exl3Error(-1, "invalid grouped EXL3 input")
        rows = x.numel() // n_in
        if rows == 0:
            raise Exl3Error(-1, "grouped EXL3 input cannot be empty")
        ys = [torch.empty(*x.shape[:-1], l.out_features, dtype=l.output_dtype(x.dtype), device=x.device)
              for l in self.linears]
        ws = self._ws.get(self.workspace_bytes(rows), x.device)
        outs = (_vp * len(ys))(*[y.data_ptr() for y in ys])
        _check(
            load_library().exl3_group_forward(
                self._handles, len(self.linears), _ptr(x), _dtype_code(x.dtype), rows, outs, _ptr(ws),
                ws.numel(), _stream_ptr(x.device),
            )
        )
        return ys

    __call__ = forward


def swiglu(gate, up):
    """Array::swiglu (native/ffi/mlx_bridge.cpp:745-749): (g * sigmoid(g)) * u in
    f16 arithmetic, for f16 device tensors of one shape."""
    torch = _torch()
    gate = _require_device(gate, "gate", (torch.float16,))
    up = _require_device(up, "up", (torch.float16,))
    if gate.shape != up.shape:
        raise Exl3Error(-1, "SwiGLU operands differ in shape")
    out = torch.empty_like(gate)
    _check(load_library().exl3_swiglu(_ptr(gate), _ptr(up), _ptr(out), gate.numel(),
                                      _stream_ptr(gate.device)))
    return out


def swiglu_down_input(gate_up, gu_svh, down_suh, selected):
    """swiglu_down_input (moe.rs:569-583) on device tensors: f32 gate_up
    [slots*2, hidden], f16 gu_svh [E, 2, hidden], f16 down_suh [E, hidden],
    int32 selected [slots] -> f16 [slots, hidden]."""
    torch = _torch()
    gate_up = _require_device(gate_up, "gate_up", (torch.float32,))
    gu_svh = _require_device(gu_svh, "gu_svh", (torch.float16,))
    down_suh = _require_device(down_suh, "down_suh", (torch.float16,))
    selected = _require_device(selected, "selected", (torch.int32,))
    hidden = gate_up.shape[-1]
    out = torch.empty(selected.numel(), hidden, dtype=torch.float16, device=gate_up.device)
    if gate_up.numel() != 2 * selected.numel() * hidden:
        raise Exl3Error(-1, "invalid fused SwiGLU dimensions")
    _check(load_library().exl3_swiglu_down_input(_ptr(gate_up), _ptr(gu_svh), _ptr(down_suh),
                                                 _ptr(selected), selected.numel(), hidden,
                                                 gu_svh.shape[0], _ptr(out),
                                                 _stream_ptr(gate_up.device)))
    return out


def finish_and_reduce(raw, svh, scores):
    """finish_and_reduce (moe.rs:586-609) on device tensors: f32 raw
    [rows*top_k, width], f16 svh of the same shape, scores [rows, top_k]
    (float16, bfloat16 or float32) -> [rows, width] in scores_result_dtype."""
    torch = _torch()
    raw = _require_device(raw, "raw", (torch.float32,))
    svh = _require_device(svh, "svh", (torch.float16,))
    scores = _require_device(scores, "scores", (torch.float16, torch.bfloat16, torch.float32))
    rows, top_k = scores.shape
    width = raw.shape[-1]
    if raw.numel() != rows * top_k * width or svh.shape != raw.shape:
        raise Exl3Error(-1, "invalid expert reduction dimensions")
    y = torch.empty(rows, width, dtype=scores_result_dtype(scores.dtype), device=raw.device)
    _check(load_library().exl3_finish_and_reduce(_ptr(raw), _ptr(svh), _ptr(scores),
                                                 _dtype_code(scores.dtype), rows, top_k, width,
                                                 _ptr(y), _stream_ptr(raw.device)))
    return y


def prepare128(x, scales):
    """The EXL3 input prologue as an op (exl3_prepare128, exl3.metal:204-216):
    f16(H128(f16(x * scales)) / sqrt(128)) per 128-column block of the f16
    rows of x; scales f16 of shape [width] (per column) or x's shape."""
    torch = _torch()
    x = _require_device(x, "x", (torch.float16,))
    scales = _require_device(scales, "scales", (torch.float16,))
    width = x.shape[-1] if x.dim() else 0
    out = torch.empty_like(x)
    _check(load_library().exl3_prepare128(_ptr(x), x.numel(), int(width), _ptr(scales),
                                          scales.numel(), _ptr(out), _stream_ptr(x.device)))
    return out


def debug_fail_launch(text: Optional[str]) -> None:
    """Arm the library's fault hook (exl3_debug_fail_launch): launches whose
    name contains `text` fail with EXL3_EDEVICE ("<name>: forced launch
    failure"); None disarms."""
    load_library().exl3_debug_fail_launch(None if text is None else text.encode())


def expert_mapped(x, trellis, suh, selected, projections: int, out: int, stride_tiles: int,
                  k: int, cb: int = 0, svh=None, raw: bool = False, workspace=None):
    """expert_mapped (linear.rs:2817-2852) over a route-major bank
    (exl3_expert_mapped): x [rows, in] (f16, bf16 or f32) with rows = routes *
    projections, trellis [in/16, bank_tiles, 16k] (int16/uint16 words), suh
    [rows, in] f16, selected [routes] (int32/uint32 expert indices); row r =
    route * projections + p multiplies tile columns selected[route] * out/16 +
    p * stride_tiles + t.  raw: the f32 products [rows, out]; else the
    output epilogue with svh [rows, out] (f16), in x's dtype."""
    torch = _torch()
    x = _require_device(x, "x", (torch.float16, torch.bfloat16, torch.float32))
    trellis = _require_device(trellis, "trellis", (torch.int16, torch.uint16))
    suh = _require_device(suh, "suh", (torch.float16,))
    selected = _require_device(selected, "selected", (torch.int32, torch.uint32))
    if x.dim() != 2 or trellis.dim() != 3 or suh.shape != x.shape or selected.dim() != 1:
        raise Exl3Error(-1, "invalid expert routes or input scales")
    rows, n_in = x.shape
    if trellis.shape[0] * 16 != n_in or trellis.shape[2] != 16 * k:
        raise Exl3Error(-1, "invalid expert trellis")
    if not raw:
        if svh is None:
            raise Exl3Error(-1, "invalid expert output scales")
        svh = _require_device(svh, "svh", (torch.float16,))
        if tuple(svh.shape) != (rows, out):
            raise Exl3Error(-1, "invalid expert output scales")
    lib = load_library()
    y = torch.empty(rows, out, dtype=torch.float32 if raw else x.dtype, device=x.device)
    need = int(lib.exl3_expert_mapped_workspace_bytes(n_in, int(out), rows))
    if workspace is None:
        workspace = torch.zeros(max(need, 1), dtype=torch.uint8, device=x.device)
    _check(lib.exl3_expert_mapped(
        _ptr(trellis), n_in, int(trellis.shape[1]), int(k), int(cb), _ptr(x), _dtype_code(x.dtype),
        rows, _ptr(suh), _ptr(selected), int(selected.numel()), int(projections), int(out),
        int(stride_tiles), None if raw else _ptr(svh), int(bool(raw)), _ptr(y), _ptr(workspace),
        workspace.numel(), _stream_ptr(x.device)))
    return y


def geglu(gate, up):
    """Array::geglu (native/ffi/mlx_bridge.cpp:764-774): the tanh GELU of gate
    times up in f16 arithmetic, for f16 device tensors of one shape."""
    torch = _torch()
    gate = _require_device(gate, "gate", (torch.float16,))
    up = _require_device(up, "up", (torch.float16,))
    if gate.shape != up.shape:
        raise Exl3Error(-1, "GEGLU operands differ in shape")
    out = torch.empty_like(gate)
    _check(load_library().exl3_geglu(_ptr(gate), _ptr(up), _ptr(out), gate.numel(),
                                     _stream_ptr(gate.device)))
    return out


class Exl3Mlp:
    """The dense SwiGLU MLP of a decoder layer (qwen35.rs:303-307: an Exl3Group
    of gate/up, Array::swiglu, the down Exl3Linear), with the SwiGLU and the
    down projection's input prologue fused into the gate/up launch."""

    def __init__(self, gate: Exl3Linear, up: Exl3Linear, down: Exl3Linear):
        if (gate.in_features, gate.out_features, gate.k, gate.cb) != \
                (up.in_features, up.out_features, up.k, up.cb):
            raise Exl3Error(-1, "incompatible grouped projections")
        if down.in_features != gate.out_features:
            raise Exl3Error(-1, f"EXL3 MLP down projection expects {down.in_features} inputs, "
                                f"gate/up give {gate.out_features}")
        self.gate, self.up, self.down = gate, up, down
        self._ws = _Workspace()

    def workspace_bytes(self, rows: int) -> int:
        return int(load_library().exl3_mlp_workspace_bytes(self.gate.handle, self.up.handle,
                                                           self.down.handle, int(rows)))

    def forward(self, x):
        torch = _torch()
        x = _require_device(x, "x", (torch.float16,))
        if x.shape[-1] != self.gate.in_features or x.numel() == 0:
            raise Exl3Error(-1, f"invalid EXL3 MLP input for {self.gate.in_features} inputs")
        rows = x.numel() // self.gate.in_features
        y = torch.empty(*x.shape[:-1], self.down.out_features, dtype=torch.float16, device=x.device)
        ws = self._ws.get(self.workspace_bytes(rows), x.device)
        _check(load_library().exl3_mlp_forward(self.gate.handle, self.up.handle, self.down.handle,
                                               _ptr(x), rows, _ptr(y), _ptr(ws), ws.numel(),
                                               _stream_ptr(x.device)))
        return y

    __call__ = forward


class Exl3SwitchGlu:
    """Exl3SwitchGlu (native/src/moe.rs:611-1153), grouped expert QMM.
    activation "silu" (new, from_checkpoint, from_lfm_checkpoint) or "gelu"
    (from_gemma_checkpoint: forward_gelu, GEGLU outputs of the columns from
    logical_hidden on set to zero; None = the whole hidden width)."""

    def __init__(self, gu_trellis, gu_suh, gu_svh, down_trellis, down_suh, down_svh, top_k: int,
                 k: int, cb: int = Codebook.DEFAULT, activation: str = "silu",
                 logical_hidden: Optional[int] = None):
        torch = _torch()
        lib = load_library()
        # Exl3SwitchGlu::new_with_activation's checks and messages (moe.rs:851-879),
        # before anything reaches the device
        if len(gu_suh.shape) != 3:
            raise Exl3Error(-1, "gate/up input scales must have rank 3")
        if len(gu_svh.shape) != 3:
            raise Exl3Error(-1, "gate/up output scales must have rank 3")
        experts, projections, n_in = (int(d) for d in gu_suh.shape)
        scale_experts, scale_projections, hidden = (int(d) for d in gu_svh.shape)
        top_k, k = int(top_k), int(k)
        if (experts <= 0 or top_k <= 0 or top_k > experts or n_in <= 0 or hidden <= 0
                or n_in % 128 or hidden % 128 or not 1 <= k <= 8 or k == 7
                or experts * hidden > 2**31 - 1 or experts * n_in > 2**31 - 1):
            raise Exl3Error(-1, "invalid or overflowing SwitchGLU dimensions")
        if projections != 2 or scale_experts != experts or scale_projections != 2:
            raise Exl3Error(-1, "invalid SwitchGLU dimensions")
        gu_tiles, down_tiles, packed = experts * hidden // 8, experts * n_in // 16, 16 * k
        if (tuple(down_suh.shape) != (experts, hidden) or tuple(down_svh.shape) != (experts, n_in)
                or tuple(gu_trellis.shape) != (n_in // 16, gu_tiles, packed)
                or tuple(down_trellis.shape) != (hidden // 16, down_tiles, packed)):
            raise Exl3Error(-1, "SwitchGLU trellis/scales disagree")
        if any(t.dtype not in (torch.int16, torch.uint16) for t in (gu_trellis, down_trellis)):
            raise Exl3Error(-1, "expert trellis must contain 16-bit integers")
        self.input, self.hidden, self.experts, self.top_k = n_in, hidden, experts, top_k
        self.k, self.cb = k, int(cb)
        if activation not in ("silu", "gelu"):
            raise Exl3Error(-1, f"unknown GLU activation {activation!r}")
        self.activation = activation
        self.logical_hidden = hidden if logical_hidden is None else int(logical_hidden)
        self.tensors = [
            _require_device(gu_trellis, "gu_trellis"),
            _require_device(gu_suh, "gu_suh").to(torch.float16).contiguous(),
            _require_device(gu_svh, "gu_svh").to(torch.float16).contiguous(),
            _require_device(down_trellis, "down_trellis"),
            _require_device(down_suh, "down_suh").to(torch.float16).contiguous(),
            _require_device(down_svh, "down_svh").to(torch.float16).contiguous(),
        ]
        h = _vp()
        if activation == "gelu":
            _check(
                lib.exl3_moe_create_gelu(
                    *[_ptr(t) for t in self.tensors], self.input, self.hidden, self.experts,
                    self.top_k, self.k, self.cb, self.logical_hidden, ctypes.byref(h),
                )
            )
        else:
            _check(
                lib.exl3_moe_create(
                    *[_ptr(t) for t in self.tensors], self.input, self.hidden, self.experts,
                    self.top_k, self.k, self.cb, ctypes.byref(h),
                )
            )
        self._handle = h
        self._ws = _Workspace()

    @classmethod
    def from_checkpoint(cls, checkpoint: "Checkpoint", prefix: str, experts: int, top_k: int,
                        names=("gate_proj", "up_proj", "down_proj"), device=None,
                        logical_hidden: Optional[int] = None) -> "Exl3SwitchGlu":
        """Exl3SwitchGlu::from_checkpoint (moe.rs:629-645, :681-800): experts
        {prefix}.{e}.{gate,up,down}, assembled into one bank on `device`
        (logical_hidden given: a GELU bank, as from_gemma_checkpoint)."""
        torch = _torch()
        device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        h = _vp()
        with torch.cuda.device(device):
            if logical_hidden is None:
                gate, up, down = (n.encode() for n in names)
                _check(load_library().exl3_moe_load(checkpoint.handle, prefix.encode(),
                                                     int(experts), int(top_k), gate, up, down,
                                                     ctypes.byref(h)))
            else:
                if tuple(names) != ("gate_proj", "up_proj", "down_proj"):
                    raise Exl3Error(-1, "GELU banks use the gate_proj/up_proj/down_proj names")
                _check(load_library().exl3_moe_load_gemma(checkpoint.handle, prefix.encode(),
                                                          int(experts), int(top_k),
                                                          int(logical_hidden), ctypes.byref(h)))
        self = cls.__new__(cls)
        self._handle = h
        self._ws = _Workspace()
        self.tensors = []  # owned by the handle
        first = checkpoint.info(f"{prefix}.0.{names[0]}.trellis")
        self.input, self.hidden = first.shape[0] * 16, first.shape[1] * 16
        self.experts, self.top_k = int(experts), int(top_k)
        self.k = first.shape[-1] // 16
        base = f"{prefix}.0.{names[0]}"
        self.cb = (Codebook.MUL1 if base + ".mul1" in checkpoint
                   else Codebook.MCG if base + ".mcg" in checkpoint else Codebook.DEFAULT)
        self.activation = "silu" if logical_hidden is None else "gelu"
        self.logical_hidden = self.hidden if logical_hidden is None else min(int(logical_hidden),
                                                                             self.hidden)
        return self

    @classmethod
    def from_gemma_checkpoint(cls, checkpoint: "Checkpoint", prefix: str, experts: int,
                              top_k: int, logical_hidden: int, device=None) -> "Exl3SwitchGlu":
        """Exl3SwitchGlu::from_gemma_checkpoint (moe.rs:663-680): GELU experts
        whose GEGLU outputs from column logical_hidden on are zero."""
        return cls.from_checkpoint(checkpoint, prefix, experts, top_k, device=device,
                                   logical_hidden=logical_hidden)

    @classmethod
    def from_lfm_checkpoint(cls, checkpoint: "Checkpoint", prefix: str, experts: int, top_k: int,
                            device=None) -> "Exl3SwitchGlu":
        """Exl3SwitchGlu::from_lfm_checkpoint (moe.rs:647-661): w1/w3/w2 experts."""
        return cls.from_checkpoint(checkpoint, prefix, experts, top_k, ("w1", "w3", "w2"), device)

    def __del__(self):
        h = getattr(self, "_handle", None)
        if h is not None and h.value and _lib is not None:
            _lib.exl3_moe_destroy(h)
            self._handle = None

    def forward(self, x, selected, scores):
        """Exl3SwitchGlu::forward (moe.rs:905-975): x [rows, in] (float16,
        bfloat16 or float32; cast to f16 as routed_inputs reads it), selected
        [rows, top_k] expert ids, scores [rows, top_k] (float16, bfloat16 or
        float32, kept in their dtype) -> [rows, in] in scores_result_dtype."""
        torch = _torch()
        floats = (torch.float16, torch.bfloat16, torch.float32)
        x = _require_device(x, "x", floats)
        rows = x.shape[0]
        if x.dim() != 2 or x.shape[1] != self.input or tuple(selected.shape) != (rows, self.top_k) \
                or tuple(scores.shape) != (rows, self.top_k):
            raise Exl3Error(-1, "invalid SwitchGLU input/routes")
        selected = _require_device(selected, "selected").to(torch.int32).contiguous()
        scores = _require_device(scores, "scores", floats)
        y = torch.empty(rows, self.input, dtype=scores_result_dtype(scores.dtype), device=x.device)
        need = int(load_library().exl3_moe_workspace_bytes(self._handle, rows))
        ws = self._ws.get(need, x.device)
        _check(
            load_library().exl3_moe_forward(
                self._handle, _ptr(x), _dtype_code(x.dtype), rows, _ptr(selected), _ptr(scores),
                _dtype_code(scores.dtype), _ptr(y), _ptr(ws), ws.numel(), _stream_ptr(x.device),
            )
        )
        return y

    __call__ = forward


def pack_tiles(states, k: int):
    """Trellis tiles of 256-state blocks on the GPU (the `metal-pack` codec op,
    exl3.metal:85-100): int16/uint16 device tensor of whole tiles -> int16
    tensor of 16*k words per tile."""
    torch = _torch()
    states = _require_device(states, "states")
    if states.element_size() != 2:
        raise Exl3Error(-1, "states must be 16-bit integers")
    if states.numel() % 256:
        raise Exl3Error(-1, "expected whole 256-state tiles")
    tiles = states.numel() // 256
    out = torch.empty(tiles * 16 * int(k), dtype=torch.int16, device=states.device)
    _check(load_library().exl3_pack_tiles(_ptr(states), tiles, int(k), _ptr(out),
                                          _stream_ptr(states.device)))
    return out


def codewords(states, cb: int):
    """f16 codewords of arbitrary 16-bit states (the `codebook` codec op,
    codec.rs:52-71) on the GPU: int16/uint16 device tensor -> float16."""
    torch = _torch()
    states = _require_device(states, "states")
    values = torch.empty(states.shape, dtype=torch.float16, device=states.device)
    _check(load_library().exl3_codewords(_ptr(states), states.numel(), int(cb), _ptr(values),
                                         _stream_ptr(states.device)))
    return values


def qmv_inner(packed, x, cols: int, k: int, cb: int):
    """The serial inner QMV without glue (the `metal-qmv` codec op, exl3.metal:118-142):
    y[n] = f16(sum_r x[r] W[r][n]) for a packed [rows/16][cols/16][16k] trellis."""
    torch = _torch()
    packed = _require_device(packed, "packed")
    x = _require_device(x, "x", (torch.float16,))
    rows = x.numel()
    y = torch.empty(cols, dtype=torch.float16, device=x.device)
    need = int(load_library().exl3_qmv_inner_workspace_bytes(rows, int(cols)))
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=x.device)
    _check(load_library().exl3_qmv_inner(_ptr(packed), rows, int(cols), int(k), int(cb), _ptr(x),
                                         _ptr(y), _ptr(ws), ws.numel(), _stream_ptr(x.device)))
    return y


def decode_tiles(packed, k: int, cb: int, with_states: bool = True):
    """Decode every tile of a packed trellis on the GPU.

    packed: device int16/uint16 tensor whose size is a multiple of 16*k.
    Returns (states uint16 [tiles, 256] or None, values float16 [tiles, 256])
    in each tile's stored (permuted) order.
    """
    torch = _torch()
    packed = _require_device(packed, "packed")
    if not (1 <= int(k) <= 8):
        raise Exl3Error(-1, f"K must be in 1..=8, got {k}")
    if packed.numel() % (16 * k):
        raise Exl3Error(-1, "packed length is not a whole tile")
    tiles = packed.numel() // (16 * k)
    values = torch.empty(tiles, 256, dtype=torch.float16, device=packed.device)
    states = torch.empty(tiles, 256, dtype=torch.uint16, device=packed.device) if with_states else None
    _check(
        load_library().exl3_decode_tiles(
            _ptr(packed), tiles, int(k), int(cb), _ptr(states), _ptr(values), _stream_ptr(packed.device)
        )
    )
    return states, values
