"""The C-ABI library loads and exports what include/exl3_hip.h declares, and
host-side validation rejects bad arguments before any launch (no GPU needed:
none of these calls reaches the device)."""

import ctypes
import re
from pathlib import Path

import pytest

import mlxl3_amd
from mlxl3_amd import LIB_PATH, EXPORTED_SYMBOLS

HEADER = Path(__file__).resolve().parent.parent / "include" / "exl3_hip.h"

pytestmark = pytest.mark.skipif(not LIB_PATH.exists(), reason="libexl3_hip.so not built")


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(exl3_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    lib = ctypes.CDLL(str(LIB_PATH))
    names = declared_functions()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(EXPORTED_SYMBOLS) == names


def test_version_and_empty_error():
    lib = mlxl3_amd.load_library()
    assert b"gfx950" in lib.exl3_version()
    assert isinstance(lib.exl3_last_error(), bytes)


FAKE = 0x1000  # never dereferenced by create


def create(k=4, cb=0, n_in=256, n_out=256, trellis=FAKE, suh=FAKE, svh=FAKE):
    lib = mlxl3_amd.load_library()
    h = ctypes.c_void_p()
    rc = lib.exl3_linear_create(trellis, n_in, n_out, k, cb, suh, svh, None, ctypes.byref(h))
    return rc, h, lib.exl3_last_error().decode()


@pytest.mark.parametrize(
    "kwargs,msg",
    [
        (dict(k=0), "K must be in 1..=8, got 0"),
        (dict(k=9), "K must be in 1..=8, got 9"),
        (dict(cb=3), "invalid EXL3 codebook 3"),
        (dict(n_in=192), "128-aligned"),
        (dict(n_out=100), "128-aligned"),
        (dict(trellis=None), "null weight pointer"),
        # 65536 x 65536 at K=8: 4 GiB of trellis, past the 32-bit kernel offsets
        (dict(k=8, n_in=65536, n_out=65536), "exceeds the 4 GiB limit"),
    ],
)
def test_create_rejects_like_the_reference(kwargs, msg):
    rc, h, err = create(**kwargs)
    assert rc == -1 and not h.value
    assert msg in err


def test_create_and_workspace_sizes():
    lib = mlxl3_amd.load_library()
    rc, h, _ = create(n_in=4096, n_out=14336)
    assert rc == 0 and h.value
    try:
        assert lib.exl3_linear_in_features(h) == 4096
        assert lib.exl3_linear_out_features(h) == 14336
        ws1 = lib.exl3_linear_workspace_bytes(h, 1)
        ws16 = lib.exl3_linear_workspace_bytes(h, 16)
        ws512 = lib.exl3_linear_workspace_bytes(h, 512)
        assert 0 < ws1 < ws16
        assert ws512 >= 512 * 4096 * 2
        assert lib.exl3_linear_workspace_bytes(h, 0) == 0
    finally:
        lib.exl3_linear_destroy(h)


def test_forward_rejects_before_launch():
    lib = mlxl3_amd.load_library()
    rc, h, _ = create()
    try:
        # rows < 1
        assert lib.exl3_linear_forward(h, FAKE, 9, 0, FAKE, 9, FAKE, 1 << 20, None) == -1
        assert "empty" in lib.exl3_last_error().decode()
        # bad dtype
        assert lib.exl3_linear_forward(h, FAKE, 7, 1, FAKE, 9, FAKE, 1 << 20, None) == -1
        # workspace too small
        assert lib.exl3_linear_forward(h, FAKE, 9, 1, FAKE, 9, FAKE, 4, None) == -1
        assert "workspace too small" in lib.exl3_last_error().decode()
        # null activations
        assert lib.exl3_linear_forward(h, None, 9, 1, FAKE, 9, FAKE, 1 << 20, None) == -1
    finally:
        lib.exl3_linear_destroy(h)


def test_output_dtype_follows_mlx_promotion():
    """linear.rs:992-995: y.astype(x.dtype) + an f16 bias under MLX's promotion:
    bf16 + f16 is f32, so a biased projection under bf16 activations returns
    f32; without a bias the activation dtype comes back.  forward rejects any
    other y_type before a launch."""
    lib = mlxl3_amd.load_library()
    plain = ctypes.c_void_p()
    biased = ctypes.c_void_p()
    assert lib.exl3_linear_create(FAKE, 256, 256, 4, 0, FAKE, FAKE, None, ctypes.byref(plain)) == 0
    assert lib.exl3_linear_create(FAKE, 256, 256, 4, 0, FAKE, FAKE, FAKE, ctypes.byref(biased)) == 0
    try:
        for x_type in (9, 10, 12):
            assert lib.exl3_linear_output_dtype(plain, x_type) == x_type
        assert [lib.exl3_linear_output_dtype(biased, t) for t in (9, 10, 12)] == [9, 10, 10]
        assert lib.exl3_linear_output_dtype(biased, 7) == -1
        assert lib.exl3_linear_output_dtype(None, 9) == -1
        for h, x_type, y_type in ((biased, 12, 12), (plain, 12, 10), (plain, 9, 10)):
            assert lib.exl3_linear_forward(h, FAKE, x_type, 1, FAKE, y_type, FAKE, 1 << 20,
                                           None) == -1
            msg = lib.exl3_last_error().decode()
            assert f"EXL3 output dtype {y_type} differs" in msg, msg
    finally:
        lib.exl3_linear_destroy(plain)
        lib.exl3_linear_destroy(biased)


def test_decode_rejects_bad_k_and_cb():
    lib = mlxl3_amd.load_library()
    assert lib.exl3_decode_tiles(FAKE, 1, 0, 0, None, FAKE, None) == -1
    assert lib.exl3_decode_tiles(FAKE, 1, 4, 5, None, FAKE, None) == -1
    assert lib.exl3_decode_tiles(FAKE, 0, 4, 0, None, FAKE, None) == 0  # nothing to do


def test_group_rejects_mismatched_members():
    lib = mlxl3_amd.load_library()
    rc1, a, _ = create(n_in=256)
    rc2, b, _ = create(n_in=512)
    try:
        parts = (ctypes.c_void_p * 2)(a.value, b.value)
        ys = (ctypes.c_void_p * 2)(FAKE, FAKE)
        assert lib.exl3_group_forward(parts, 2, FAKE, 9, 1, ys, FAKE, 1 << 20, None) == -1
        assert "same input width" in lib.exl3_last_error().decode()
    finally:
        lib.exl3_linear_destroy(a)
        lib.exl3_linear_destroy(b)


def moe_create(n_in=256, hidden=256, experts=8, top_k=2, k=3, cb=0, ptr=FAKE):
    lib = mlxl3_amd.load_library()
    h = ctypes.c_void_p()
    rc = lib.exl3_moe_create(ptr, ptr, ptr, ptr, ptr, ptr, n_in, hidden, experts, top_k, k, cb,
                             ctypes.byref(h))
    return rc, h, lib.exl3_last_error().decode()


@pytest.mark.parametrize(
    "kwargs,msg",
    [
        # switch_glu_layout (native/src/contracts.rs:4-28) and its unit test
        (dict(k=7), "invalid or overflowing SwitchGLU dimensions"),
        (dict(k=0), "invalid or overflowing SwitchGLU dimensions"),
        (dict(k=9), "invalid or overflowing SwitchGLU dimensions"),
        (dict(experts=2, top_k=3), "invalid or overflowing SwitchGLU dimensions"),
        (dict(top_k=0), "invalid or overflowing SwitchGLU dimensions"),
        (dict(n_in=127), "invalid or overflowing SwitchGLU dimensions"),
        (dict(hidden=0), "invalid or overflowing SwitchGLU dimensions"),
        (dict(experts=2**31 - 1, top_k=1), "invalid or overflowing SwitchGLU dimensions"),
        (dict(cb=3), "invalid EXL3 codebook 3"),
        (dict(ptr=None), "SwitchGLU trellis/scales disagree"),
    ],
)
def test_moe_create_rejects_like_the_reference(kwargs, msg):
    rc, h, err = moe_create(**kwargs)
    assert rc == -1 and not h.value and msg in err


def test_moe_create_workspace_and_forward_rejects():
    lib = mlxl3_amd.load_library()
    rc, h, err = moe_create()
    assert rc == 0 and h.value, err
    try:
        one = lib.exl3_moe_workspace_bytes(h, 1)
        many = lib.exl3_moe_workspace_bytes(h, 100)
        assert 0 < one < many
        assert lib.exl3_moe_workspace_bytes(h, 0) == 0
        # rows < 1, null routes, short workspace: rejected before any launch
        assert lib.exl3_moe_forward(h, FAKE, 9, 0, FAKE, FAKE, 9, FAKE, FAKE, one, None) == -1
        assert lib.exl3_moe_forward(h, FAKE, 9, 1, None, FAKE, 9, FAKE, FAKE, one, None) == -1
        assert "invalid SwitchGLU input/routes" in lib.exl3_last_error().decode()
        # activation and score dtypes: f16, bf16 or f32 only
        assert lib.exl3_moe_forward(h, FAKE, 11, 1, FAKE, FAKE, 9, FAKE, FAKE, one, None) == -1
        assert "unsupported dtype codes 11 (x), 9 (scores)" in lib.exl3_last_error().decode()
        assert lib.exl3_moe_forward(h, FAKE, 12, 1, FAKE, FAKE, 3, FAKE, FAKE, one, None) == -1
        assert "unsupported dtype codes 12 (x), 3 (scores)" in lib.exl3_last_error().decode()
        assert lib.exl3_moe_forward(h, FAKE, 10, 100, FAKE, FAKE, 12, FAKE, FAKE, one, None) == -1
        assert "workspace too small" in lib.exl3_last_error().decode()
        assert lib.exl3_moe_in_features(h) == 256 and lib.exl3_moe_hidden_features(h) == 256
        assert lib.exl3_moe_in_features(None) == 0
    finally:
        lib.exl3_moe_destroy(h)


def test_moe_create_gelu_validates_the_logical_width():
    """forward_gelu zeroes GEGLU outputs from logical_hidden on (moe.rs:1125-1137):
    widths <= 0 are rejected, widths past hidden zero nothing; the bank checks
    are those of exl3_moe_create (K=7 has no SwitchGLU layout, contracts.rs:51)."""
    lib = mlxl3_amd.load_library()

    def gelu_create(logical, k=3):
        h = ctypes.c_void_p()
        rc = lib.exl3_moe_create_gelu(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 256, 256, 8, 2, k, 0,
                                      logical, ctypes.byref(h))
        return rc, h, lib.exl3_last_error().decode()

    for logical in (0, -128):
        rc, h, err = gelu_create(logical)
        assert rc == -1 and not h.value and "invalid logical GLU width" in err
    rc, h, err = gelu_create(128, k=7)
    assert rc == -1 and not h.value and "invalid or overflowing SwitchGLU dimensions" in err
    for logical in (1, 200, 256, 4096):
        rc, h, err = gelu_create(logical)
        assert rc == 0 and h.value, err
        assert lib.exl3_moe_workspace_bytes(h, 3) > 0
        lib.exl3_moe_destroy(h)


def test_geglu_rejects_before_launch():
    lib = mlxl3_amd.load_library()
    assert lib.exl3_geglu(FAKE, FAKE, FAKE, -1, None) == -1
    assert "negative element count" in lib.exl3_last_error().decode()
    assert lib.exl3_geglu(None, FAKE, FAKE, 8, None) == -1
    assert "null GEGLU buffer" in lib.exl3_last_error().decode()
    assert lib.exl3_geglu(None, None, None, 0, None) == 0


def test_standalone_ops_reject_before_launch():
    lib = mlxl3_amd.load_library()
    err = lambda: lib.exl3_last_error().decode()
    # prepare128_blocks (contracts.rs:2146-2159)
    for elements, width, scales in ((128, 127, 127), (641, 640, 640), (1920, 640, 1919), (0, 0, 0)):
        assert lib.exl3_prepare128(FAKE, elements, width, FAKE, scales, FAKE, None) == -1
        assert "expected complete 128-aligned rows and column or element scales" in err()
    assert lib.exl3_prepare128(None, 0, 128, None, 0, None, None) == 0
    assert lib.exl3_pack_tiles(FAKE, 1, 0, FAKE, None) == -1 and "K must be in 1..=8" in err()
    assert lib.exl3_pack_tiles(None, 0, 3, None, None) == 0
    assert lib.exl3_swiglu_down_input(FAKE, FAKE, FAKE, FAKE, 4, 100, 2, FAKE, None) == -1
    assert "invalid fused SwiGLU dimensions" in err()
    assert lib.exl3_swiglu_down_input(FAKE, None, FAKE, FAKE, 4, 128, 2, FAKE, None) == -1
    assert "invalid fused SwiGLU scales/routes" in err()
    assert lib.exl3_finish_and_reduce(FAKE, FAKE, FAKE, 9, 2, 2, 100, FAKE, None) == -1
    assert "invalid expert reduction dimensions" in err()
    assert lib.exl3_finish_and_reduce(FAKE, FAKE, FAKE, 9, 2, 0, 128, FAKE, None) == -1
    assert lib.exl3_finish_and_reduce(FAKE, FAKE, FAKE, 11, 2, 2, 128, FAKE, None) == -1
    assert "unsupported score dtype code 11" in err()


def test_group_and_mlp_reject_before_launch():
    lib = mlxl3_amd.load_library()
    hs = [create(n_in=256, n_out=256)[1] for _ in range(9)]
    d_bad = create(n_in=512, n_out=256)[1]
    g_k = create(k=3, n_in=256, n_out=256)[1]
    try:
        parts = (ctypes.c_void_p * 9)(*[h.value for h in hs])
        ys = (ctypes.c_void_p * 9)(*([FAKE] * 9))
        assert lib.exl3_group_forward(parts, 9, FAKE, 9, 1, ys, FAKE, 1 << 20, None) == -4
        assert "more than 8" in lib.exl3_last_error().decode()
        assert lib.exl3_group_workspace_bytes(parts, 9, 1) == 0
        assert lib.exl3_group_workspace_bytes(parts, 8, 1) > lib.exl3_group_workspace_bytes(parts, 1, 1)
        assert lib.exl3_group_forward(parts, 0, FAKE, 9, 1, ys, FAKE, 1 << 20, None) == -1
        # workspace sized for one member is too small for eight
        small = lib.exl3_group_workspace_bytes(parts, 1, 4)
        assert lib.exl3_group_forward(parts, 8, FAKE, 9, 4, ys, FAKE, small, None) == -1
        assert "workspace too small" in lib.exl3_last_error().decode()
        # MLP: gate/up must match, down.in == gate.out, f16 only
        a, b = hs[0], hs[1]
        assert lib.exl3_mlp_forward(a, g_k, b, FAKE, 1, FAKE, FAKE, 1 << 24, None) == -1
        assert "incompatible grouped projections" in lib.exl3_last_error().decode()
        assert lib.exl3_mlp_forward(a, b, d_bad, FAKE, 1, FAKE, FAKE, 1 << 24, None) == -1
        assert "down projection expects 512 inputs" in lib.exl3_last_error().decode()
        assert lib.exl3_mlp_workspace_bytes(a, b, d_bad, 1) == 0
        need = lib.exl3_mlp_workspace_bytes(a, b, hs[2], 40)
        assert need > 65536
        assert lib.exl3_mlp_forward(a, b, hs[2], FAKE, 40, FAKE, FAKE, need - 1, None) == -1
        assert "workspace too small" in lib.exl3_last_error().decode()
        assert lib.exl3_mlp_forward(a, b, hs[2], FAKE, 0, FAKE, FAKE, need, None) == -1
        assert lib.exl3_swiglu(FAKE, FAKE, FAKE, -1, None) == -1
        assert lib.exl3_swiglu(None, None, None, 0, None) == 0
    finally:
        for h in hs + [d_bad, g_k]:
            lib.exl3_linear_destroy(h)


def _switch_args(experts=4, n_in=256, hidden=128, k=3, top_k=2, **over):
    """CPU tensors of a valid SwitchGLU bank's shapes (moe.rs:851-879)."""
    import torch

    a = dict(
        gu_trellis=torch.zeros(n_in // 16, experts * hidden // 8, 16 * k, dtype=torch.int16),
        gu_suh=torch.zeros(experts, 2, n_in, dtype=torch.float16),
        gu_svh=torch.zeros(experts, 2, hidden, dtype=torch.float16),
        down_trellis=torch.zeros(hidden // 16, experts * n_in // 16, 16 * k, dtype=torch.int16),
        down_suh=torch.zeros(experts, hidden, dtype=torch.float16),
        down_svh=torch.zeros(experts, n_in, dtype=torch.float16),
        top_k=top_k, k=k)
    a.update(over)
    return a


@pytest.mark.parametrize(
    "over,msg",
    [
        (dict(gu_suh="rank2"), "gate/up input scales must have rank 3"),
        (dict(gu_svh="rank2"), "gate/up output scales must have rank 3"),
        (dict(k=7), "invalid or overflowing SwitchGLU dimensions"),
        (dict(top_k=5), "invalid or overflowing SwitchGLU dimensions"),
        (dict(gu_suh=(4, 3, 256)), "invalid SwitchGLU dimensions"),
        (dict(gu_svh=(3, 2, 128)), "invalid SwitchGLU dimensions"),
        (dict(down_suh=(4, 256)), "SwitchGLU trellis/scales disagree"),
        (dict(down_svh=(4, 128)), "SwitchGLU trellis/scales disagree"),
        (dict(gu_trellis=(16, 64, 32)), "SwitchGLU trellis/scales disagree"),
        (dict(down_trellis=(8, 64, 32)), "SwitchGLU trellis/scales disagree"),
        (dict(k=2), "SwitchGLU trellis/scales disagree"),  # last dimension 16*k
        (dict(down_trellis="int32"), "expert trellis must contain 16-bit integers"),
    ],
)
def test_switch_glu_constructor_rejects_like_the_reference(over, msg):
    """Exl3SwitchGlu::new_with_activation's checks (moe.rs:851-879) run in the
    Python mirror before any tensor reaches the device or the C ABI."""
    import torch

    base = _switch_args()
    args = dict(base)
    for name, v in over.items():
        if v == "rank2":
            args[name] = base[name].reshape(base[name].shape[0], -1)
        elif v == "int32":
            args[name] = base[name].to(torch.int32)
        elif isinstance(v, tuple):
            args[name] = torch.zeros(v, dtype=base[name].dtype)
        else:
            args[name] = v
    with pytest.raises(mlxl3_amd.Exl3Error) as e:
        mlxl3_amd.Exl3SwitchGlu(**args)
    assert msg in str(e.value), str(e.value)


def test_switch_glu_constructor_accepts_valid_shapes_then_needs_a_device():
    with pytest.raises(mlxl3_amd.Exl3Error) as e:
        mlxl3_amd.Exl3SwitchGlu(**_switch_args())
    assert "must be a device tensor" in str(e.value)
