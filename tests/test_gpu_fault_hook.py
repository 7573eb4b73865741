"""The launch fault hook on the GPU: a failure forced after earlier kernels of a
call ran (the MoE's gate/up launch, the QMM path's prologue launch) returns
EXL3_EDEVICE with the launch's message, leaves the output untouched (the
kernels that write it are never launched) and the workspace valid: the same
call, disarmed, then gives the result of a fresh workspace bit for bit."""

import numpy as np
import pytest

import mlxl3_amd
from mlxl3_amd import synth

pytestmark = pytest.mark.gpu


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


def test_moe_failure_after_gate_up_keeps_output_and_workspace():
    torch = torch_mod()
    print("fault hook: moe gate/up", flush=True)
    in_f, hidden, E, top_k, k, rows = 256, 256, 8, 2, 3, 24
    layer = synth.moe_layer(9, 100, in_f, hidden, E, k)
    bank = [dev(a) for a in layer]
    moe = mlxl3_amd.Exl3SwitchGlu(bank[0], bank[1], bank[2], bank[3], bank[4], bank[5],
                                  top_k=top_k, k=k, cb=0)
    x = dev(synth.activations(9, 1, rows, in_f))
    sel, sc = synth.moe_routes(9, 2, rows, E, top_k)
    sel, sc = dev(sel), dev(sc)
    lib = mlxl3_amd.load_library()
    nws = int(lib.exl3_moe_workspace_bytes(moe._handle, rows))
    ws = torch.zeros(nws, dtype=torch.uint8, device="cuda")
    y = torch.full((rows, in_f), 7.0, dtype=torch.float16, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    mlxl3_amd.debug_fail_launch("moe gate/up")
    try:
        rc = lib.exl3_moe_forward(moe._handle, x.data_ptr(), 9, rows, sel.data_ptr(),
                                  sc.data_ptr(), 9, y.data_ptr(), ws.data_ptr(), nws, stream)
        err = lib.exl3_last_error().decode()
    finally:
        mlxl3_amd.debug_fail_launch(None)
    torch.cuda.synchronize()
    assert rc == -2 and err == "moe gate/up: forced launch failure", (rc, err)
    assert bool((y == 7.0).all())
    rc = lib.exl3_moe_forward(moe._handle, x.data_ptr(), 9, rows, sel.data_ptr(), sc.data_ptr(),
                              9, y.data_ptr(), ws.data_ptr(), nws, stream)
    assert rc == 0
    fresh = torch.zeros(nws, dtype=torch.uint8, device="cuda")
    y2 = torch.empty_like(y)
    assert lib.exl3_moe_forward(moe._handle, x.data_ptr(), 9, rows, sel.data_ptr(),
                                sc.data_ptr(), 9, y2.data_ptr(), fresh.data_ptr(), nws,
                                stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))


def test_qmm_failure_after_prologue_keeps_output_and_workspace():
    torch = torch_mod()
    print("fault hook: QMM prologue", flush=True)
    rows, n_in, n_out, k = 40, 512, 384, 4
    tr, suh, svh, _ = synth.linear_layer(31, 0, n_in, n_out, k)
    lin = mlxl3_amd.Exl3Linear(dev(tr), dev(suh), dev(svh), None, k, 0)
    x = dev(synth.activations(31, 1, rows, n_in))
    ws = torch.zeros(lin.workspace_bytes(rows), dtype=torch.uint8, device="cuda")
    mlxl3_amd.debug_fail_launch("EXL3 prologue")
    try:
        with pytest.raises(mlxl3_amd.Exl3Error, match="EXL3 prologue launch: forced launch failure"):
            lin.forward(x, workspace=ws)
    finally:
        mlxl3_amd.debug_fail_launch(None)
    y = lin.forward(x, workspace=ws)
    y_fresh = lin.forward(x)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y_fresh.view(torch.int16))
