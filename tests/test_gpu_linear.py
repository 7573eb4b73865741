"""GPU EXL3 linear (QMV for M <= 16, QMM above) through the C ABI, against
the CPU oracle on the same seeded inputs.

Tolerances (stated, measured on MI355X):
* vs the oracle in engine glue semantics (mode 1), which differs from the GPU
  only in the f32 summation order of the inner product: max-abs <= 2 f16 ulp
  of max|y|, relative L2 <= 1e-3.  A 1-ulp flip of one f16(yhat) value can
  move several outputs of its 128-block through the two interior f16 roundings
  of the Hadamard, so the exact-match fraction is reported, not bounded;
* basis rows (the reference's one-hot QMV check, check-metal-tiles.py.txt):
  with suh = 1 and x = 2^-3 * (a Sylvester row), xhat is one-hot, every inner
  product is one exact f16 x f16 product, and the output must be bit-exact;
* vs ref/forward.py semantics (mode 0, f32 Hadamards): relative L2 <= 2e-3,
  max-abs <= 8 f16 ulp of max|y|.
Bit-exact properties: rows of one call equal the same rows alone (batch ==
serial) within each kernel family.
"""

import numpy as np
import pytest

import oracle
from mlxl3_amd import synth

pytestmark = pytest.mark.gpu

TOL_MODE1_REL = 1e-3
MIN_EXACT_MODE1 = 0.0
TOL_MODE1_ULP = 2
TOL_MODE0_REL = 2e-3
TOL_MODE0_ULP = 8


def torch_mod():
    import torch

    return torch


def make_layer(seed, n_in, n_out, k, cb, bias=False):
    import mlxl3_amd

    torch = torch_mod()
    tr, suh, svh, b = synth.linear_layer(seed, 10, n_in, n_out, k, bias=bias)
    dev = lambda a: torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).cuda()
    lin = mlxl3_amd.Exl3Linear(dev(tr), dev(suh), dev(svh), None if b is None else dev(b), k, cb)
    return lin, (tr, suh, svh, b)


def run(lin, x_np, dtype=None):
    torch = torch_mod()
    x = torch.from_numpy(x_np).cuda()
    if dtype is not None:
        x = x.to(dtype)
    y = lin.forward(x)
    torch.cuda.synchronize()
    return y


def stats(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    rel = np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-30)
    ulp = float(np.spacing(np.float16(np.abs(ref).max())))
    return rel, np.abs(y - ref).max() / ulp


def check(y, ref, rel_tol, ulp_tol, label, min_exact=0.0):
    rel, ulps = stats(y, ref)
    exact = float(np.mean(np.asarray(y) == np.asarray(ref)))
    print(f"{label}: rel_l2={rel:.3e} max_abs={ulps:.2f} ulp(max|y|) exact={exact:.4f}", flush=True)
    assert rel <= rel_tol and ulps <= ulp_tol and exact >= min_exact, (label, rel, ulps, exact)


@pytest.mark.parametrize("k", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_qmv_small_all_k_cb(k, cb):
    print(f"qmv k={k} cb={cb}", flush=True)
    lin, (tr, suh, svh, _) = make_layer(1000 + 10 * k + cb, 512, 384, k, cb)
    x = synth.activations(3, k, 1, 512)
    y = run(lin, x).cpu().numpy()
    ref1 = oracle.forward(x, tr, suh, svh, k, cb, mode=1)
    ref0 = oracle.forward(x, tr, suh, svh, k, cb, mode=0)
    check(y, ref1, TOL_MODE1_REL, TOL_MODE1_ULP, f"k{k} cb{cb} vs mode1", MIN_EXACT_MODE1)
    check(y, ref0, TOL_MODE0_REL, TOL_MODE0_ULP, f"k{k} cb{cb} vs mode0")


@pytest.mark.parametrize("rows", [1, 2, 3, 5, 8, 13, 16])
def test_qmv_rows_vs_oracle_and_batch_equals_serial(rows):
    torch = torch_mod()
    print(f"qmv rows={rows}", flush=True)
    lin, (tr, suh, svh, _) = make_layer(2000 + rows, 1024, 768, 4, 0)
    x = synth.activations(4, rows, rows, 1024)
    y = run(lin, x).cpu().numpy()
    check(y, oracle.forward(x, tr, suh, svh, 4, 0, mode=1), TOL_MODE1_REL, TOL_MODE1_ULP,
          f"rows{rows} vs mode1", MIN_EXACT_MODE1)
    for r in range(rows):
        yr = run(lin, x[r:r + 1]).cpu().numpy()
        assert np.array_equal(yr.view(np.uint16), y[r:r + 1].view(np.uint16)), r


def bf16_bits(v):
    """float32 -> bfloat16 bits, round to nearest even."""
    b = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def ulp_of(v, bf16):
    """Spacing of the output format at |v| (bf16: 7 fraction bits, f16 otherwise)."""
    return float(np.spacing(np.float16(v))) * (8.0 if bf16 else 1.0)


@pytest.mark.parametrize("rows, n_in", [(1, 512), (2, 512), (5, 512), (16, 512), (16, 4096),
                                         (17, 512), (512, 512)])
@pytest.mark.parametrize("dtype_name", ["bfloat16", "float32"])
@pytest.mark.parametrize("bias", [False, True])
def test_activation_dtypes_and_bias_vs_oracle(rows, n_in, dtype_name, bias):
    """bf16 / f32 activations through the QMV (rows 1, 2, 5: single-row and
    row-major exchange; 16: fragment-order exchange, with the prologue inside
    the workgroup at 512 inputs and as its own launch at 4096) and the QMM (17,
    512):
    the output dtype follows linear.rs:992-995 under MLX promotion (bf16 + f16
    bias -> f32), values vs the oracle at rel-L2 <= 1e-3 and max-abs <= 2 ulp
    at max|y| of the last format the value was rounded to (bf16 for bf16
    activations, with or without the f32 bias add: a one-ulp f16 flip in the
    inner result can move the bf16 cast by one bf16 ulp; f16 otherwise)."""
    torch = torch_mod()
    dtype = getattr(torch, dtype_name)
    print(f"dtypes rows={rows} in={n_in} {dtype_name} bias={bias}", flush=True)
    lin, (tr, suh, svh, b) = make_layer(3000 + rows + n_in, n_in, 384, 3, 1, bias=bias)
    x32 = synth.activations(5, rows, rows, n_in).astype(np.float32) * np.float32(1.37)
    xt = torch.from_numpy(x32).to(dtype)
    y = lin.forward(xt.cuda())
    torch.cuda.synchronize()
    want_dtype = torch.float32 if (bias and dtype == torch.bfloat16) else dtype
    assert y.dtype == want_dtype, (y.dtype, want_dtype)
    if dtype == torch.bfloat16:
        xb = xt.view(torch.int16).numpy().view(np.uint16)
        ref = oracle.forward(xb, tr, suh, svh, 3, 1, bias=b, x_dtype="bf16")
    else:
        ref = oracle.forward(x32, tr, suh, svh, 3, 1, bias=b)
    if ref.dtype == np.uint16:  # bf16 bits
        ref = (ref.astype(np.uint32) << 16).view(np.float32)
    got = y.float().cpu().numpy()
    bf16_out = dtype == torch.bfloat16  # the result passed through a bf16 cast
    rel = np.linalg.norm(got.astype(np.float64) - ref) / np.linalg.norm(ref.astype(np.float64))
    ulps = np.abs(got.astype(np.float64) - ref).max() / ulp_of(np.abs(ref).max(), bf16_out)
    exact = float(np.mean(got == ref))
    print(f"  rel_l2={rel:.3e} max_abs={ulps:.2f} ulp exact={exact:.4f}", flush=True)
    assert rel <= 1e-3 and ulps <= 2, (rel, ulps)


def test_bf16_bias_result_is_the_f32_sum_of_the_bf16_cast():
    """The GPU's f32 result of bf16 activations with a bias equals, bit for bit,
    float32(its own bias-free bf16 output) + float32(bias): the cast happens
    before the promoted add (linear.rs:993-995), in both kernel families."""
    torch = torch_mod()
    import mlxl3_amd

    lin_b, (tr, suh, svh, b) = make_layer(3100, 512, 384, 4, 0, bias=True)
    lin_n = mlxl3_amd.Exl3Linear(lin_b.trellis, lin_b.suh, lin_b.svh, None, 4, 0)
    for rows in (3, 40):
        x = torch.from_numpy(synth.activations(6, rows, rows, 512)).to(torch.bfloat16).cuda()
        yb, yn = lin_b.forward(x), lin_n.forward(x)
        torch.cuda.synchronize()
        assert yb.dtype == torch.float32 and yn.dtype == torch.bfloat16
        want = yn.float() + torch.from_numpy(b.astype(np.float32)).cuda()
        assert torch.equal(yb, want), rows


@pytest.mark.parametrize("rows", [17, 64, 130, 512])
@pytest.mark.parametrize("k,cb", [(4, 0), (3, 0), (5, 1), (2, 2)])
def test_qmm_vs_oracle(rows, k, cb):
    print(f"qmm rows={rows} k={k} cb={cb}", flush=True)
    lin, (tr, suh, svh, _) = make_layer(4000 + rows + k, 512, 512, k, cb)
    x = synth.activations(6, rows, rows, 512, outlier_frac=0.01)
    y = run(lin, x).cpu().numpy()
    check(y, oracle.forward(x, tr, suh, svh, k, cb, mode=1), TOL_MODE1_REL, TOL_MODE1_ULP,
          f"qmm rows{rows} vs mode1", MIN_EXACT_MODE1)


def sylvester_row(i):
    j = np.arange(128)
    return np.where(np.bitwise_count(i & j) % 2, -1.0, 1.0)


def basis_inputs(rows, n_in, seed):
    """x rows whose prologue output is one-hot (value f16(16/sqrt(128)))."""
    rng = np.random.default_rng(seed)
    x = np.zeros((rows, n_in), np.float16)
    picks = rng.choice(n_in, rows, replace=False)
    for r, idx in enumerate(picks):
        b, i = divmod(int(idx), 128)
        x[r, b * 128:(b + 1) * 128] = (0.125 * sylvester_row(i)).astype(np.float16)
    return x, picks


@pytest.mark.parametrize("k", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1, 2])
@pytest.mark.parametrize("rows", [16, 33])
def test_basis_rows_bit_exact(k, cb, rows):
    import mlxl3_amd

    torch = torch_mod()
    n_in, n_out = 512, 384
    tr, _, svh, _ = synth.linear_layer(8000 + k * 3 + cb, 10, n_in, n_out, k)
    suh = np.ones(n_in, np.float16)
    dev = lambda a: torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).cuda()
    lin = mlxl3_amd.Exl3Linear(dev(tr), dev(suh), dev(svh), None, k, cb)
    x, picks = basis_inputs(rows, n_in, k * 10 + cb)
    xh = oracle.prologue(x, suh).astype(np.float32)
    assert np.count_nonzero(xh) == rows and (np.abs(xh).max(1) == np.float32(np.float16(16 / np.sqrt(128)))).all()
    y = run(lin, x).cpu().numpy()
    ref = oracle.forward(x, tr, suh, svh, k, cb, mode=1)
    assert np.array_equal(y.view(np.uint16), ref.view(np.uint16)), float(np.mean(y == ref))


@pytest.mark.parametrize("kw,splits", [(1, 1), (1, 3), (2, 2), (2, 5), (4, 1), (4, 4), (1, 8)])
def test_qmv_schedules_bit_exact(kw, splits, monkeypatch):
    """Every QMV schedule (global K-splits x K-parts per workgroup) is
    bit-exact on basis rows and matches the oracle on random inputs."""
    import mlxl3_amd

    torch = torch_mod()
    monkeypatch.setenv("EXL3_QMV_KW", str(kw))
    monkeypatch.setenv("EXL3_QMV_SPLITS", str(splits))
    n_in, n_out, k, cb = 1024, 1280, 4, 0
    tr, _, svh, _ = synth.linear_layer(9000 + 10 * kw + splits, 10, n_in, n_out, k)
    suh = np.ones(n_in, np.float16)
    dev = lambda a: torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).cuda()
    lin = mlxl3_amd.Exl3Linear(dev(tr), dev(suh), dev(svh), None, k, cb)
    x, _ = basis_inputs(16, n_in, kw * 10 + splits)
    y = run(lin, x).cpu().numpy()
    assert np.array_equal(y.view(np.uint16), oracle.forward(x, tr, suh, svh, k, cb).view(np.uint16))
    xr = synth.activations(9, kw * 10 + splits, 3, n_in)
    yr = run(lin, xr).cpu().numpy()
    check(yr, oracle.forward(xr, tr, suh, svh, k, cb), TOL_MODE1_REL, TOL_MODE1_ULP,
          f"kw{kw} splits{splits}")


def test_north_star_shape_qmv():
    """4096 x 14336, K=4 3INST, batch 1 (the headline workload) vs the oracle."""
    lin, (tr, suh, svh, _) = make_layer(2, 4096, 14336, 4, 0)
    x = synth.activations(2, 0, 1, 4096)
    y = run(lin, x).cpu().numpy()
    check(y, oracle.forward(x, tr, suh, svh, 4, 0, mode=1), TOL_MODE1_REL, TOL_MODE1_ULP, "NS mode1")
    check(y, oracle.forward(x, tr, suh, svh, 4, 0, mode=0), TOL_MODE0_REL, TOL_MODE0_ULP, "NS mode0")


@pytest.mark.parametrize("rows", [2, 4, 8, 16])
def test_north_star_shape_multirow_separate_prologue(rows):
    """4096 x 14336 at M = 2, 4 (row-major exchange, fused prologue) and 8, 16
    (fragment exchange; xhat from the separate prologue launch): all of them
    launches of 3.5 waves per SIMD, so the one-slice prefetch kernels with the
    first step decoded under the prologue.  Every row must equal the same row
    run alone (the single-row kernel, M = 1) bit for bit, and the batch the
    oracle."""
    torch = torch_mod()
    lin, (tr, suh, svh, _) = make_layer(2, 4096, 14336, 4, 0)
    x = synth.activations(7, rows, rows, 4096)
    y = run(lin, x).cpu().numpy()
    for r in (0, rows // 2, rows - 1):
        yr = run(lin, x[r:r + 1]).cpu().numpy()
        assert np.array_equal(y[r:r + 1].view(np.uint16), yr.view(np.uint16)), r
    check(y, oracle.forward(x, tr, suh, svh, 4, 0, mode=1), TOL_MODE1_REL, TOL_MODE1_ULP,
          f"NS M={rows} mode1")
    del torch


@pytest.mark.parametrize("n_in, n_out", [(4096, 14336), (14336, 4096)])
@pytest.mark.parametrize("k", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_full_shape_every_k_and_codebook(n_in, n_out, k, cb):
    """Both NS-sized shapes for every K x codebook at 1, 4 and 16 rows
    (single-row, row-major and fragment-order exchanges; 16 rows take xhat
    from the prologue launch).  4096 x 14336 puts 3.5 waves on a SIMD, so it
    runs the one-slice prefetch kernels with the first step decoded under the
    prologue (for 16 % K != 0 the second set's loads issued before it);
    14336 x 4096 (1.75 waves) the two-slice ones.  Basis rows bit-exact
    against the oracle, random rows within the stated tolerance, and rows of
    a batch equal to the same rows run alone."""
    import mlxl3_amd

    torch = torch_mod()
    print(f"full shape {n_in}x{n_out} k={k} cb={cb}", flush=True)
    tr, _, svh, _ = synth.linear_layer(11000 + 10 * k + cb, 10, n_in, n_out, k)
    suh = np.ones(n_in, np.float16)
    dev = lambda a: torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).cuda()
    lin = mlxl3_amd.Exl3Linear(dev(tr), dev(suh), dev(svh), None, k, cb)
    for rows in (1, 4, 16):
        x, _ = basis_inputs(rows, n_in, 100 * k + 10 * cb + rows)
        y = run(lin, x).cpu().numpy()
        ref = oracle.forward(x, tr, suh, svh, k, cb, mode=1)
        assert np.array_equal(y.view(np.uint16), ref.view(np.uint16)), \
            (k, cb, rows, float(np.mean(y == ref)))
        xr = synth.activations(12, 10 * k + cb, rows, n_in)
        yr = run(lin, xr).cpu().numpy()
        check(yr, oracle.forward(xr, tr, suh, svh, k, cb, mode=1), TOL_MODE1_REL, TOL_MODE1_ULP,
              f"{n_in}x{n_out} k{k} cb{cb} M={rows}")
        for r in ((0, rows - 1) if rows > 1 else ()):
            y1 = run(lin, xr[r:r + 1]).cpu().numpy()
            assert np.array_equal(yr[r:r + 1].view(np.uint16), y1.view(np.uint16)), (k, cb, rows, r)


def test_qmm_rows_independent_of_batch():
    lin, _ = make_layer(5000, 512, 384, 4, 0)
    x = synth.activations(7, 0, 300, 512)
    y_all = run(lin, x).cpu().numpy()
    y_part = run(lin, x[:40]).cpu().numpy()
    assert np.array_equal(y_all[:40].view(np.uint16), y_part.view(np.uint16))


def test_group_equals_separate():
    import mlxl3_amd

    a, _ = make_layer(6000, 512, 256, 4, 0)
    b, _ = make_layer(6001, 512, 384, 4, 0)
    g = mlxl3_amd.Exl3Group([a, b])
    torch = torch_mod()
    for rows in (1, 7, 40):
        x = torch.from_numpy(synth.activations(8, rows, rows, 512)).cuda()
        ys = g.forward(x)
        torch.cuda.synchronize()
        for lin, y in zip((a, b), ys):
            assert torch.equal(y, lin.forward(x))


def test_c1_full_size_qmv():
    """C1: 4096x4096 K4 3INST, batch 1, vs the oracle."""
    lin, (tr, suh, svh, _) = make_layer(1, 4096, 4096, 4, 0)
    x = synth.activations(1, 0, 1, 4096)
    y = run(lin, x).cpu().numpy()
    check(y, oracle.forward(x, tr, suh, svh, 4, 0, mode=1), TOL_MODE1_REL, TOL_MODE1_ULP, "C1 mode1",
          MIN_EXACT_MODE1)
    check(y, oracle.forward(x, tr, suh, svh, 4, 0, mode=0), TOL_MODE0_REL, TOL_MODE0_ULP, "C1 mode0")


@pytest.mark.parametrize("rows", [1, 5, 16, 17, 40])
@pytest.mark.parametrize("k,cb", [(4, 0), (2, 1), (3, 2)])
def test_smallest_shape(rows, k, cb):
    """in = out = 128: one Hadamard block, one column block, one K-split, on
    both sides of the QMV/QMM boundary (M = 16 / 17)."""
    lin, (tr, suh, svh, _) = make_layer(6200 + rows + k, 128, 128, k, cb)
    x = synth.activations(10, rows + k, rows, 128)
    y = run(lin, x).cpu().numpy()
    check(y, oracle.forward(x, tr, suh, svh, k, cb, mode=1), TOL_MODE1_REL, TOL_MODE1_ULP,
          f"128x128 M={rows} k{k} cb{cb}")


def test_qmm_long_prefill_rows():
    """NS shape at M = 4096 (16 row tiles of 256 rows, 1792 workgroups): rows at
    the start, a tile boundary and the end vs the oracle."""
    lin, (tr, suh, svh, _) = make_layer(6300, 4096, 14336, 4, 0)
    rows = 4096
    x = synth.activations(11, 0, rows, 4096, outlier_frac=0.01)
    y = run(lin, x).cpu().numpy()
    assert np.isfinite(y).all()
    pick = np.array([0, 255, 256, 2049, rows - 1])
    check(y[pick], oracle.forward(x[pick], tr, suh, svh, 4, 0, mode=1), TOL_MODE1_REL,
          TOL_MODE1_ULP, f"NS M={rows} rows {pick.tolist()}")


def test_invalid_input_raises_without_launch():
    import mlxl3_amd

    torch = torch_mod()
    lin, _ = make_layer(7000, 256, 256, 4, 0)
    with pytest.raises(mlxl3_amd.Exl3Error):
        lin.forward(torch.zeros(1, 128, dtype=torch.float16, device="cuda"))
    with pytest.raises(mlxl3_amd.Exl3Error):
        lin.forward(torch.zeros(0, 256, dtype=torch.float16, device="cuda"))


@pytest.mark.parametrize("n_in,n_out,rows,k,cb", [
    (4096, 14336, 1, 4, 0), (4096, 14336, 4, 4, 0), (14336, 4096, 1, 4, 0),
    (4096, 4096, 1, 3, 0), (4096, 4096, 1, 5, 1), (2048, 6144, 2, 2, 2),
])
def test_repeat_calls_bit_identical(n_in, n_out, rows, k, cb):
    """Regression: the decode writes the MFMA B fragments with inline assembly,
    which the compiler's hazard recognizer does not see, so a schedule with one
    wait state between the last half-write of a fragment and its MFMA fed the
    MFMA the register's previous value.  That showed as outputs that changed
    from call to call (the second tile of each column pair) while staying close
    to the oracle.  Five calls of one input must agree bit for bit, and the
    first must match the oracle."""
    lin, (tr, suh, svh, _) = make_layer(31 + k, n_in, n_out, k, cb)
    x = synth.activations(5, rows, rows, n_in)
    ys = [run(lin, x).cpu().numpy() for _ in range(5)]
    for i, y in enumerate(ys[1:], 1):
        assert np.array_equal(ys[0].view(np.uint16), y.view(np.uint16)), i
    check(ys[0], oracle.forward(x, tr, suh, svh, k, cb, mode=1), TOL_MODE1_REL, TOL_MODE1_ULP,
          f"{n_in}x{n_out} rows{rows} K{k} cb{cb} repeat")


@pytest.mark.parametrize("n_in,n_out,rows", [
    (4096, 14336, 1), (4096, 14336, 4), (4096, 14336, 16), (14336, 4096, 1),
    (4096, 4096, 2), (14336, 4096, 512),
])
def test_split_exchange_alternating_inputs(n_in, n_out, rows):
    """The split-K exchange (partials through coherent stores, an arrival
    counter, the last arriver's coherent loads) relies on acknowledged stores
    being visible before the counter increment.  A partial read before its
    store landed would be the previous call's, so calls alternate between two
    inputs on one workspace (the previous call's partials always differ): 60
    calls, each bit-identical to its input's first result.  Shapes: the
    single-row, row-major, fragment-order and QMM (4 K-splits) exchanges."""
    torch = torch_mod()
    lin, _ = make_layer(4100 + rows, n_in, n_out, 4, 0)
    xs = [torch.from_numpy(synth.activations(60 + i, rows, rows, n_in)).cuda() for i in range(2)]
    ws = torch.zeros(lin.workspace_bytes(rows), dtype=torch.uint8, device="cuda")
    want = [lin.forward(x, workspace=ws).clone() for x in xs]
    torch.cuda.synchronize()
    assert not torch.equal(want[0], want[1])
    outs = [lin.forward(xs[i % 2], workspace=ws) for i in range(60)]
    torch.cuda.synchronize()
    for i, y in enumerate(outs):
        assert torch.equal(y.view(torch.int16), want[i % 2].view(torch.int16)), i

