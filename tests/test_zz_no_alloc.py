"""exl3_linear_forward_noalloc: the allocation-free variant of
exl3_linear_forward (its workspace is a fixed device array of the library).

Through the C ABI: the output equals exl3_linear_forward's bit for bit on two
calls in a row, the second with a smaller input (the array keeps the first
call's contents, so stale scratch must not leak into the second); both kernel
families (QMV rows <= 16, QMM above) and the split-K paths whose counters live
in the array.  Calls needing more workspace than the array holds are rejected
before any device work (checked without a GPU)."""

import ctypes

import numpy as np
import pytest

import mlxl3_amd
from mlxl3_amd import synth

pytestmark = pytest.mark.skipif(not mlxl3_amd.LIB_PATH.exists(), reason="library not built")


def test_noalloc_rejects_oversized_calls_before_device_work():
    lib = mlxl3_amd.load_library()
    h = ctypes.c_void_p()
    assert lib.exl3_linear_create(0x1000, 4096, 14336, 4, 0, 0x1000, 0x1000, None,
                                  ctypes.byref(h)) == 0
    try:
        cap = lib.exl3_linear_noalloc_max_bytes()
        assert cap >= (32 << 20)
        rows = 1
        while lib.exl3_linear_workspace_bytes(h, rows) <= cap:
            rows *= 2
        rc = lib.exl3_linear_forward_noalloc(h, 0x1000, 9, rows, 0x1000, 9, None)
        assert rc == -4
        msg = lib.exl3_last_error().decode()
        assert f"allocation-free EXL3 forward of {rows} rows needs" in msg, msg
        assert lib.exl3_linear_forward_noalloc(h, 0x1000, 9, 0, 0x1000, 9, None) == -1
        assert lib.exl3_linear_forward_noalloc(None, 0x1000, 9, 1, 0x1000, 9, None) == -1
    finally:
        lib.exl3_linear_destroy(h)


@pytest.mark.gpu
@pytest.mark.parametrize("n_in,n_out,k,cb,rows", [
    (4096, 14336, 4, 0, (16, 1)),     # QMV split-K, then the single-row kernel
    (1024, 768, 3, 1, (300, 40)),     # QMM, then a smaller QMM
    (14336, 4096, 2, 2, (130, 7)),    # QMM with global split-K, then the multi-row QMV
])
def test_noalloc_equals_workspace_forward_on_two_calls(n_in, n_out, k, cb, rows):
    import torch

    print(f"noalloc {n_in}x{n_out} k={k} cb={cb} rows={rows}", flush=True)
    lib = mlxl3_amd.load_library()
    tr, suh, svh, b = synth.linear_layer(77, 1, n_in, n_out, k, bias=True)
    dev = lambda a: torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).cuda()
    lin = mlxl3_amd.Exl3Linear(dev(tr), dev(suh), dev(svh), dev(b), k, cb)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for m in rows:
        x = torch.from_numpy(synth.activations(9, m, m, n_in)).cuda()
        want = lin.forward(x)
        y = torch.empty_like(want)
        rc = lib.exl3_linear_forward_noalloc(lin.handle, x.data_ptr(), 9, m, y.data_ptr(), 9,
                                             stream)
        assert rc == 0, lib.exl3_last_error().decode()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16)), m
