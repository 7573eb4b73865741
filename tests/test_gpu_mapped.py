"""exl3_expert_mapped (expert_mapped, linear.rs:2817-2852) on the GPU and the
codec's mlx-expert op (main.rs:540-597), against the oracle's expert_mapped
(pinned to the oracle's linear forward in test_oracle_mapped.py):

* every K (not 7) x codebook, 1-3 projections per route with a projection
  stride, f16 / bf16 / f32 activations, the epilogue and raw f32 outputs:
  rel L2 <= 1e-3 and max-abs <= 2 f16 ulp of max|y| (the linear's bar; raw:
  rel L2 <= 1e-3);
* rows are independent: each row computed alone equals its row of the batch
  bit for bit, and a route whose expert leaves the bank gives zero rows;
* the decode shape of a SwitchGLU layer (1 token x top-8 x gate/up over a
  128-expert bank, 2048 -> 768, K=3), and the same gate/up bank driven as the
  SwitchGLU's gate and up projections (stride = experts * 768/16);
* mlx-expert answers the ABI's words (f16) and values (f32) exactly, and the
  reference's request errors.
"""

import numpy as np
import pytest

import oracle
from codec_client import run

pytestmark = pytest.mark.gpu

TOL_REL = 1e-3
TOL_ULP = 2


def torch_mod():
    import torch

    return torch


def check(y, ref, label, ulp=True):
    y = np.asarray(y, np.float64)
    r = np.asarray(ref, np.float64)
    rel = np.linalg.norm(y - r) / np.linalg.norm(r)
    ulps = np.abs(y - r).max() / float(np.spacing(np.float16(np.abs(r).max())))
    print(f"{label}: rel_l2={rel:.3e} max_abs={ulps:.2f} ulp", flush=True)
    assert rel <= TOL_REL and (not ulp or ulps <= TOL_ULP), (label, rel, ulps)


def case(seed, k, in_f, out, experts, projections, stride, routes):
    rng = np.random.default_rng(seed)
    ot = out // 16
    tiles = (experts - 1) * ot + (projections - 1) * stride + ot
    bank = rng.integers(0, 1 << 16, (in_f // 16, tiles, 16 * k), dtype=np.uint16)
    rows = routes * projections
    selected = rng.integers(0, experts, routes).astype(np.uint32)
    suh = ((rng.random((rows, in_f)) + 0.5) * np.where(rng.random((rows, in_f)) < 0.5, -1, 1)
           ).astype(np.float16)
    svh = ((rng.random((rows, out)) + 0.5) / np.sqrt(in_f)).astype(np.float16)
    x = rng.normal(0, 1, (rows, in_f)).astype(np.float16)
    return bank, selected, suh, svh, x


def dev(a):
    torch = torch_mod()
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def gpu(x, bank, suh, selected, projections, out, stride, k, cb, svh=None, raw=False):
    import mlxl3_amd

    torch = torch_mod()
    y = mlxl3_amd.expert_mapped(x, dev(bank), dev(suh), dev(selected), projections, out, stride,
                                k, cb, svh=None if svh is None else dev(svh), raw=raw)
    torch.cuda.synchronize()
    return y.cpu()


@pytest.mark.parametrize("k", [1, 2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_mapped_vs_oracle(k, cb):
    torch = torch_mod()
    projections, stride = (k % 3) + 1, 24
    bank, sel, suh, svh, x = case(500 + 10 * k + cb, k, 512, 256, 6, projections, stride, 3)
    print(f"mapped k={k} cb={cb} P={projections}", flush=True)
    y = gpu(torch.from_numpy(x).cuda(), bank, suh, sel, projections, 256, stride, k, cb, svh=svh)
    check(y.numpy(), oracle.expert_mapped(x, suh, bank, sel, projections, 256, stride, k, cb,
                                          svh=svh), f"mapped k={k} cb={cb}")
    raw = gpu(torch.from_numpy(x).cuda(), bank, suh, sel, projections, 256, stride, k, cb, raw=True)
    check(raw.numpy(), oracle.expert_mapped(x, suh, bank, sel, projections, 256, stride, k, cb,
                                            raw=True), f"mapped raw k={k} cb={cb}", ulp=False)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_mapped_activation_dtypes(dtype):
    torch = torch_mod()
    bank, sel, suh, svh, x16 = case(77, 4, 256, 128, 4, 2, 8, 4)
    if dtype == "bf16":
        xt = torch.from_numpy(x16).cuda().to(torch.bfloat16)
        xo, kw = xt.view(torch.int16).cpu().numpy().view(np.uint16), {"x_dtype": "bf16"}
    else:
        xt = torch.from_numpy(x16).cuda().float() * 1.001
        xo, kw = xt.cpu().numpy(), {}
    y = gpu(xt, bank, suh, sel, 2, 128, 8, 4, 0, svh=svh)
    ref = oracle.expert_mapped(xo, suh, bank, sel, 2, 128, 8, 4, 0, svh=svh, **kw)
    if dtype == "bf16":
        assert y.dtype == torch.bfloat16
        got = y.view(torch.int16).numpy().view(np.uint16).astype(np.uint32) << 16
        want = ref.astype(np.uint32) << 16
        check(got.view(np.float32), want.view(np.float32), "mapped bf16", ulp=False)
    else:
        assert y.dtype == torch.float32
        check(y.numpy(), ref, "mapped f32")


def test_mapped_rows_are_independent_and_bank_checked():
    torch = torch_mod()
    bank, sel, suh, svh, x = case(91, 3, 256, 128, 4, 2, 8, 5)
    sel[2] = 99  # past the bank: zero rows 4 and 5
    xt = torch.from_numpy(x).cuda()
    y = gpu(xt, bank, suh, sel, 2, 128, 8, 3, 1, svh=svh).numpy()
    assert not y[4:6].any() and y[:4].any() and y[6:].any()
    ref = oracle.expert_mapped(x, suh, bank, sel, 2, 128, 8, 3, 1, svh=svh)
    assert not ref[4:6].any()
    for route in (0, 3):
        rows = slice(2 * route, 2 * route + 2)
        alone = gpu(xt[rows].contiguous(), bank, suh[rows], sel[route:route + 1], 2, 128, 8, 3, 1,
                    svh=svh[rows]).numpy()
        assert np.array_equal(alone.view(np.uint16), y[rows].view(np.uint16)), route


def test_mapped_switchglu_decode_shape():
    """1 token x top-8 over the gate/up bank of a 128-expert SwitchGLU (2048 ->
    768, K=3): rows = 8 routes x 2 projections, up tiles at stride E * 48."""
    torch = torch_mod()
    E, in_f, hidden, k = 128, 2048, 768, 3
    rng = np.random.default_rng(12)
    ot = hidden // 16
    bank = rng.integers(0, 1 << 16, (in_f // 16, 2 * E * ot, 16 * k), dtype=np.uint16)
    sel = rng.choice(E, 8, replace=False).astype(np.uint32)
    rows = 16
    x = np.repeat(rng.normal(0, 1, (1, in_f)).astype(np.float16), rows, axis=0)
    suh = ((rng.random((rows, in_f)) + 0.5)).astype(np.float16)
    raw = gpu(torch.from_numpy(x).cuda(), bank, suh, sel, 2, hidden, E * ot, k, 0, raw=True)
    ref = oracle.expert_mapped(x, suh, bank, sel, 2, hidden, E * ot, k, 0, raw=True)
    check(raw.numpy(), ref, "mapped decode shape", ulp=False)


def test_mapped_abi_errors():
    import mlxl3_amd

    torch = torch_mod()
    bank, sel, suh, svh, x = case(5, 2, 256, 128, 3, 1, 0, 2)
    xt = torch.from_numpy(x).cuda()
    for kw, msg in (
        (dict(k=7), "mapped K=7 is not supported"),
        (dict(out=120), "expert output width must be 128-aligned"),
        (dict(projections=3), "expert route count does not match input rows"),
        (dict(projections=2, routes=1, stride=1000), "expert tile map outside the bank"),
    ):
        args = dict(projections=1, out=128, stride=0, k=2, routes=2)
        args.update(kw)
        kk = args["k"]
        tr = bank if kk == 2 else np.zeros((16, bank.shape[1], 16 * kk), np.uint16)
        with pytest.raises(mlxl3_amd.Exl3Error, match=msg):
            mlxl3_amd.expert_mapped(xt, dev(tr), dev(suh), dev(sel[:args["routes"]]),
                                    args["projections"], args["out"], args["stride"], kk, 0,
                                    raw=True)


def test_mlx_expert_codec_op():
    torch = torch_mod()
    bank, sel, suh, svh, x = case(33, 4, 256, 128, 5, 2, 16, 3)
    base = {"op": "mlx-expert", "k": 4, "mode": 2, "projections_per_route": 2,
            "projection_stride_tiles": 16, "cols": 128, "selected": sel.tolist(),
            "x": x.view(np.uint16).ravel().tolist(), "data": bank.ravel().tolist(),
            "suh": suh.view(np.uint16).ravel().tolist()}
    reqs = [
        {**base, "svh": svh.view(np.uint16).ravel().tolist()},
        {**base, "return_raw": True},
        {**base, "k": 7, "svh": svh.view(np.uint16).ravel().tolist()},
        {**base, "projections_per_route": 0},
        {**base, "selected": []},
        {**base, "x": [0] * 7},
        {**base, "k": 0},
    ]
    rows = run(reqs)
    xt = torch.from_numpy(x).cuda()
    y = gpu(xt, bank, suh, sel, 2, 128, 16, 4, 2, svh=svh).numpy()
    raw = gpu(xt, bank, suh, sel, 2, 128, 16, 4, 2, raw=True).numpy()
    assert rows[0] == {"data": {"f16": y.view(np.uint16).ravel().tolist()}}
    got = np.asarray(rows[1]["data"]["f32"], np.float32)
    assert np.array_equal(got.view(np.uint32), raw.ravel().view(np.uint32))
    assert rows[2] == {"error": "mapped K=7 is not supported"}
    assert rows[3] == {"error": "invalid projection count"}
    assert rows[4] == {"error": "missing expert routes"}
    assert "error" in rows[5]
    assert rows[6] == {"error": "K must be in 1..=8, got 0"}
