"""Grouped projections in one launch, the SwiGLU op and the fused SwiGLU MLP on
the GPU, through the C ABI.

* exl3_group_forward (Exl3Group::forward, native/src/linear.rs:2285-2382): one
  launch over all members' column blocks (rows <= 16) or one prologue + one QMM
  launch; every member's output must be bit-identical to its own
  exl3_linear_forward (same kernels, same split order per column block);
* exl3_swiglu (Array::swiglu, native/ffi/mlx_bridge.cpp:745-749) against the
  oracle's f16-staged restatement: bit-exact for every finite f16 gate value;
* exl3_mlp_forward (qwen35.rs:303-307; rows <= 16: SwiGLU in the gate/up QMV
  epilogue, which also applies the down projection's prologue where down would
  otherwise launch it separately; rows > 16: one SwiGLU + down-prologue kernel
  between the QMMs)
  against the unfused composition
  exl3_group_forward -> exl3_swiglu -> exl3_linear_forward: bit-exact; and
  against the oracle composition (oracle.mlp_forward) within the linear's
  stated tolerance chain (rel L2 <= 2e-3, max-abs <= 1e-2 of rms(y): the
  oracle's summation order differs, and a 1-ulp flip of a gate/up value
  propagates through the SwiGLU and the down projection).
"""

import numpy as np
import pytest

import oracle
from mlxl3_amd import synth

pytestmark = pytest.mark.gpu


def torch_mod():
    import torch

    return torch


def dev(a):
    torch = torch_mod()
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def make(seed, tid, n_in, n_out, k, cb, bias=False, svh_scale=1.0):
    import mlxl3_amd

    tr, suh, svh, b = synth.linear_layer(seed, tid, n_in, n_out, k, bias=bias)
    if svh_scale != 1.0:
        svh = (svh.astype(np.float32) * svh_scale).astype(np.float16)
    lin = mlxl3_amd.Exl3Linear(dev(tr), dev(suh), dev(svh), None if b is None else dev(b), k, cb)
    return lin, (tr, suh, svh, b, k, cb)


def same_bits(a, b):
    torch = torch_mod()
    if a.dtype != b.dtype or a.shape != b.shape:
        return False
    as_int = torch.int16 if a.element_size() == 2 else torch.int32
    return bool(torch.equal(a.contiguous().view(as_int), b.contiguous().view(as_int)))


@pytest.mark.parametrize("k, cb", [(2, 0), (4, 1), (3, 2), (8, 0), (5, 1), (6, 2), (7, 0)])
@pytest.mark.parametrize("rows", [1, 5, 16, 17, 64, 200])
def test_group_one_launch_equals_separate(k, cb, rows):
    import mlxl3_amd

    torch = torch_mod()
    print(f"group k={k} cb={cb} rows={rows}", flush=True)
    widths = [512, 128, 256]  # q / k / v-like members of unequal width
    lins = [make(80 + i, 20 + i, 384, w, k, cb, bias=(i == 1))[0] for i, w in enumerate(widths)]
    group = mlxl3_amd.Exl3Group(lins)
    x = torch.from_numpy(synth.activations(90 + rows, 5, rows, 384)).cuda()
    ys = group.forward(x)
    singles = [lin.forward(x) for lin in lins]
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(ys, singles)):
        assert a.shape == (rows, widths[i])
        assert same_bits(a, b), (k, cb, rows, i)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_group_dtypes_and_eight_members(dtype):
    import mlxl3_amd

    torch = torch_mod()
    lins = [make(3, 40 + i, 256, 128 * (1 + i % 3), 4, 0)[0] for i in range(8)]
    group = mlxl3_amd.Exl3Group(lins)
    for rows in (3, 33):
        x = torch.from_numpy(synth.activations(7, 1, rows, 256)).cuda().to(getattr(torch, dtype))
        ys = group.forward(x)
        singles = [lin.forward(x) for lin in lins]
        torch.cuda.synchronize()
        for a, b in zip(ys, singles):
            assert a.dtype == x.dtype and same_bits(a, b)


def test_swiglu_all_f16_gates():
    import mlxl3_amd

    torch = torch_mod()
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    g = bits.view(np.float16)
    g = np.tile(g[np.isfinite(g)], 2)
    u = (np.random.default_rng(3).standard_normal(g.size) * 3).astype(np.float16)
    ref = oracle.swiglu(g, u)
    for off in (0, 1):  # aligned (8-wide path) and unaligned (scalar path) buffers
        gd, ud = dev(g[off:]), dev(u[off:])
        out = mlxl3_amd.swiglu(gd, ud)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        r = ref[off:]
        nan = np.isnan(r)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint16), r[~nan].view(np.uint16)), off


def mlp_case(n_in, hidden, k, cb, seed=11):
    import mlxl3_amd

    fan = 1.0 / np.sqrt(n_in)
    gate, gp = make(seed, 1, n_in, hidden, k, cb, svh_scale=fan)
    up, upp = make(seed, 2, n_in, hidden, k, cb, svh_scale=fan)
    down, dp = make(seed, 3, hidden, n_in, k, cb, svh_scale=1.0 / np.sqrt(hidden))
    return mlxl3_amd.Exl3Mlp(gate, up, down), (gate, up, down), (gp, upp, dp)


def unfused(parts, x):
    import mlxl3_amd

    gate, up, down = parts
    g, u = mlxl3_amd.Exl3Group([gate, up]).forward(x)
    return down.forward(mlxl3_amd.swiglu(g, u))


def check_tol(y, ref, label):
    y64, r64 = y.astype(np.float64), ref.astype(np.float64)
    rel = np.linalg.norm(y64 - r64) / np.linalg.norm(r64)
    mx = np.abs(y64 - r64).max() / np.sqrt(np.mean(r64 ** 2))
    print(f"{label}: rel_l2={rel:.3e} max_abs/rms={mx:.3e}", flush=True)
    assert rel <= 2e-3 and mx <= 1e-2, (label, rel, mx)


@pytest.mark.parametrize("k, cb", [(4, 0), (2, 1), (3, 2)])
@pytest.mark.parametrize("rows", [1, 3, 16, 17, 100, 300])
def test_mlp_fused_equals_unfused_and_oracle(k, cb, rows):
    torch = torch_mod()
    print(f"mlp k={k} cb={cb} rows={rows}", flush=True)
    mlp, parts, host = mlp_case(256, 384, k, cb)
    x_np = synth.activations(60 + rows, 3, rows, 256)
    x = torch.from_numpy(x_np).cuda()
    y = mlp.forward(x)
    y_ref = unfused(parts, x)
    torch.cuda.synchronize()
    assert same_bits(y, y_ref), (k, cb, rows)
    if rows <= 100:
        check_tol(y.cpu().numpy(), oracle.mlp_forward(x_np, *host), f"mlp k={k} cb={cb} rows={rows}")


@pytest.mark.parametrize("hidden, rows, k, cb", [(8192, 16, 4, 0), (20480, 4, 4, 0),
                                                 (8192, 16, 3, 2), (8192, 16, 2, 1),
                                                 (20480, 4, 5, 1)])
def test_mlp_separate_prologue_rows(hidden, rows, k, cb):
    """4096 -> hidden -> 4096 where the down projection would take its xhat
    from a prologue launch of its own (16 rows x 4-block K-ranges; 4 rows x 160
    blocks x 32 column blocks = 20 480 repeated jobs): the fused MLP's gate/up
    epilogue writes down's xhat instead, and the unfused path runs the
    prologue launch; fused == unfused bit-exact."""
    torch = torch_mod()
    print(f"mlp separate prologue hidden={hidden} rows={rows} k={k} cb={cb}", flush=True)
    mlp, parts, _ = mlp_case(4096, hidden, k, cb, seed=9)
    x = torch.from_numpy(synth.activations(3, rows, rows, 4096)).cuda()
    y = mlp.forward(x)
    y_ref = unfused(parts, x)
    torch.cuda.synchronize()
    assert same_bits(y, y_ref)


@pytest.mark.parametrize("rows", [5, 1100])
def test_mlp_wide_intermediate(rows):
    """A wide intermediate (512 column blocks of 128) through both paths."""
    torch = torch_mod()
    mlp, parts, _ = mlp_case(128, 65536, 2, 0, seed=5)
    x = torch.from_numpy(synth.activations(9, rows, rows, 128)).cuda()
    y = mlp.forward(x)
    y_ref = unfused(parts, x)
    torch.cuda.synchronize()
    assert same_bits(y, y_ref)


def test_mlp_repeated_calls_share_workspace():
    """Counters are left at zero: alternating MLP, group and linear calls on
    one workspace give the same bits as fresh calls."""
    import mlxl3_amd

    torch = torch_mod()
    mlp, (gate, up, down), _ = mlp_case(256, 384, 4, 0)
    lib = mlxl3_amd.load_library()
    need = max(mlp.workspace_bytes(300), gate.workspace_bytes(300), 1 << 20)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    outs = {}
    for it in range(2):
        for rows in (2, 300):
            x = torch.from_numpy(synth.activations(rows, 4, rows, 256)).cuda()
            y = torch.empty(rows, 256, dtype=torch.float16, device="cuda")
            s = torch.cuda.current_stream().cuda_stream
            rc = lib.exl3_mlp_forward(gate.handle, up.handle, down.handle, x.data_ptr(), rows,
                                      y.data_ptr(), ws.data_ptr(), need, s)
            assert rc == 0, lib.exl3_last_error()
            yl = torch.empty(rows, 384, dtype=torch.float16, device="cuda")
            rc = lib.exl3_linear_forward(gate.handle, x.data_ptr(), 9, rows, yl.data_ptr(), 9,
                                         ws.data_ptr(), need, s)
            assert rc == 0, lib.exl3_last_error()
            torch.cuda.synchronize()
            key = rows
            if it == 0:
                outs[key] = (y.clone(), yl.clone())
            else:
                assert same_bits(y, outs[key][0]) and same_bits(yl, outs[key][1])
    # and the counter region is zero again
    torch.cuda.synchronize()
    assert int(ws[:65536].view(torch.int32).abs().sum().item()) == 0
