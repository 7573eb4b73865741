"""The library's launch fault hook (exl3_debug_fail_launch, EXL3_FAIL_LAUNCH),
which plays the part of a failing launch caught by the reference's protect()
(native/ffi/mlx_bridge.cpp:56-66): on the CPU, with host buffers standing in
for device memory (the entry points validate, then the armed gate fails before
any HIP call), every armed entry point returns EXL3_EDEVICE with
"<launch>: forced launch failure" as its thread's message and writes nothing to
its output; an unmatched text leaves validation errors untouched; NULL disarms.
The GPU side (a failure after earlier kernels ran, the workspace still usable
for the next call) is in test_gpu_fault_hook.py."""

import ctypes
import subprocess
import sys

import numpy as np
import pytest

import mlxl3_amd

EDEVICE = -2
F16 = 9


@pytest.fixture()
def lib():
    L = mlxl3_amd.load_library()
    yield L
    L.exl3_debug_fail_launch(None)


def ptr(a):
    return a.ctypes.data


def make_linear(L, n_in, n_out, k=2):
    tr = np.zeros((n_in // 16, n_out // 16, 16 * k), np.uint16)
    suh = np.ones(n_in, np.float16)
    svh = np.ones(n_out, np.float16)
    h = ctypes.c_void_p()
    assert L.exl3_linear_create(ptr(tr), n_in, n_out, k, 0, ptr(suh), ptr(svh), None,
                                ctypes.byref(h)) == 0
    return h, (tr, suh, svh)


def expect_forced(L, rc, launch):
    assert rc == EDEVICE, rc
    assert L.exl3_last_error().decode() == f"{launch}: forced launch failure"


@pytest.mark.parametrize("rows, launch", [(1, "EXL3 QMV launch"), (40, "EXL3 QMM launch")])
def test_linear_forward_fails_before_any_write(lib, rows, launch):
    h, keep = make_linear(lib, 256, 128)
    x = np.ones((rows, 256), np.float16)
    y = np.full((rows, 128), 0x7E01, np.uint16)  # sentinel
    ws = np.zeros(int(lib.exl3_linear_workspace_bytes(h, rows)), np.uint8)
    lib.exl3_debug_fail_launch(b"EXL3 Q")
    rc = lib.exl3_linear_forward(h, ptr(x), F16, rows, ptr(y), F16, ptr(ws), ws.size, None)
    expect_forced(lib, rc, launch)
    assert (y == 0x7E01).all() and not ws.any()
    # the same call with a bad output dtype still fails validation first
    rc = lib.exl3_linear_forward(h, ptr(x), F16, rows, ptr(y), 10, ptr(ws), ws.size, None)
    assert rc == -1 and "output dtype" in lib.exl3_last_error().decode()
    lib.exl3_linear_destroy(h)


def test_group_mlp_prepare_and_glu_fail_when_armed(lib):
    g, kg = make_linear(lib, 256, 128)
    u, ku = make_linear(lib, 256, 128)
    d, kd = make_linear(lib, 128, 256)
    x = np.ones((1, 256), np.float16)
    y = np.full((1, 256), 0x7E01, np.uint16)
    lib.exl3_debug_fail_launch(b"launch")
    parts = (ctypes.c_void_p * 2)(g.value, u.value)
    outs = (ctypes.c_void_p * 2)(ptr(y), ptr(y))
    ws = np.zeros(int(lib.exl3_group_workspace_bytes(parts, 2, 1)), np.uint8)
    expect_forced(lib, lib.exl3_group_forward(parts, 2, ptr(x), F16, 1, outs, ptr(ws), ws.size,
                                              None), "EXL3 QMV launch")
    ws = np.zeros(int(lib.exl3_mlp_workspace_bytes(g, u, d, 1)), np.uint8)
    expect_forced(lib, lib.exl3_mlp_forward(g, u, d, ptr(x), 1, ptr(y), ptr(ws), ws.size, None),
                  "EXL3 QMV launch")
    sc = np.ones(256, np.float16)
    expect_forced(lib, lib.exl3_prepare128(ptr(x), 256, 256, ptr(sc), 256, ptr(y), None),
                  "EXL3 prepare128 launch")
    expect_forced(lib, lib.exl3_swiglu(ptr(x), ptr(x), ptr(y), 256, None), "SwiGLU launch")
    expect_forced(lib, lib.exl3_geglu(ptr(x), ptr(x), ptr(y), 256, None), "GEGLU launch")
    assert (y == 0x7E01).all()
    for h in (g, u, d):
        lib.exl3_linear_destroy(h)


def test_moe_and_expert_mapped_fail_when_armed(lib):
    E, n_in, hidden, top_k, k = 4, 128, 128, 2, 2
    gu = np.zeros((n_in // 16, 2 * E * hidden // 16, 16 * k), np.uint16)
    dn = np.zeros((hidden // 16, E * n_in // 16, 16 * k), np.uint16)
    ones = lambda *s: np.ones(s, np.float16)  # noqa: E731
    gsu, gsv, dsu, dsv = ones(E, 2, n_in), ones(E, 2, hidden), ones(E, hidden), ones(E, n_in)
    h = ctypes.c_void_p()
    assert lib.exl3_moe_create(ptr(gu), ptr(gsu), ptr(gsv), ptr(dn), ptr(dsu), ptr(dsv), n_in,
                               hidden, E, top_k, k, 0, ctypes.byref(h)) == 0
    rows = 3
    x = ones(rows, n_in)
    sel = np.array([[0, 1], [2, 3], [1, 2]], np.uint32)
    scores = ones(rows, top_k)
    y = np.full((rows, n_in), 0x7E01, np.uint16)
    ws = np.zeros(int(lib.exl3_moe_workspace_bytes(h, rows)), np.uint8)
    lib.exl3_debug_fail_launch(b"moe")
    # 6 routed slots take the small-row path: gate/up is its first launch
    expect_forced(lib, lib.exl3_moe_forward(h, ptr(x), F16, rows, ptr(sel), ptr(scores), F16,
                                            ptr(y), ptr(ws), ws.size, None), "moe gate/up")
    assert (y == 0x7E01).all() and not ws.any()
    # 66 slots take the grouped path: the route plan is its first launch
    big = 33
    xb, yb = ones(big, n_in), np.full((big, n_in), 0x7E01, np.uint16)
    selb, scb = np.tile(sel, (11, 1)), ones(big, top_k)
    wsb = np.zeros(int(lib.exl3_moe_workspace_bytes(h, big)), np.uint8)
    expect_forced(lib, lib.exl3_moe_forward(h, ptr(xb), F16, big, ptr(selb), ptr(scb), F16,
                                            ptr(yb), ptr(wsb), wsb.size, None), "moe plan")
    assert (yb == 0x7E01).all() and not wsb.any()
    lib.exl3_moe_destroy(h)
    # the mapped expert QMV
    bank = np.zeros((n_in // 16, E * 8, 16 * k), np.uint16)
    suh = ones(rows, n_in)
    ym = np.full((rows, 128), 0x7E01, np.uint16)
    wsm = np.zeros(int(lib.exl3_expert_mapped_workspace_bytes(n_in, 128, rows)), np.uint8)
    routes = np.array([0, 3, 1], np.uint32)
    lib.exl3_debug_fail_launch(b"expert")
    rc = lib.exl3_expert_mapped(ptr(bank), n_in, E * 8, k, 0, ptr(x), F16, rows, ptr(suh),
                                ptr(routes), 3, 1, 128, 0, None, 1, ptr(ym), ptr(wsm), wsm.size,
                                None)
    expect_forced(lib, rc, "expert prologue")
    assert (ym == 0x7E01).all()
    # argument errors are reported before the hook is consulted
    rc = lib.exl3_expert_mapped(ptr(bank), n_in, E * 8, 7, 0, ptr(x), F16, rows, ptr(suh),
                                ptr(routes), 3, 1, 128, 0, None, 1, ptr(ym), ptr(wsm), wsm.size,
                                None)
    assert rc == -4 and lib.exl3_last_error() == b"mapped K=7 is not supported"


def test_unmatched_text_and_disarm(lib):
    h, keep = make_linear(lib, 256, 128)
    x = np.ones((1, 256), np.float16)
    y = np.zeros((1, 128), np.uint16)
    lib.exl3_debug_fail_launch(b"no launch has this name")
    # nothing armed for this entry: a too-small workspace is the error it reports
    rc = lib.exl3_linear_forward(h, ptr(x), F16, 1, ptr(y), F16, None, 0, None)
    assert rc == -1 and "workspace too small" in lib.exl3_last_error().decode()
    lib.exl3_debug_fail_launch(None)
    rc = lib.exl3_linear_forward(h, ptr(x), F16, 1, ptr(y), F16, None, 0, None)
    assert rc == -1
    lib.exl3_linear_destroy(h)


def test_environment_arms_the_hook_at_load():
    code = (
        "import ctypes, numpy as np, mlxl3_amd\n"
        "L = mlxl3_amd.load_library()\n"
        "x = np.ones(256, np.float16); y = np.zeros(256, np.uint16)\n"
        "rc = L.exl3_swiglu(x.ctypes.data, x.ctypes.data, y.ctypes.data, 256, None)\n"
        "print(rc, L.exl3_last_error().decode())\n"
    )
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                         env={**__import__("os").environ, "EXL3_FAIL_LAUNCH": "SwiGLU"},
                         timeout=120, check=True).stdout.strip().splitlines()[-1]
    assert out == "-2 SwiGLU launch: forced launch failure"
