"""Pins the CPU MoE oracle (oracle/exl3_oracle.c exl3o_moe_forward).

The reference holds no MoE output vectors, so the oracle is checked against a
second, structurally different composition built from parts that are pinned on
their own (test_oracle.py): the dense expert matrices from ``reconstruct_inner``
(golden real tiles and quantizer corpus), the f32 Hadamard (MLX fixture) and the
staged f16 schedule.  The composition slices the dense banks by column instead of
walking tiles, so a wrong bank offset, a swapped gate/up projection or a scale
taken from the wrong expert fails it; each such mistake is planted in the
composition below and must be detected.  Exact invariants: scaling every score by
2 scales y by 2 bit-for-bit (f16 and f32 are exact under powers of two), and
relabelling experts together with their banks leaves y bit-identical.
Semantics followed: Exl3SwitchGlu::forward (native/src/moe.rs:905-975),
routed_inputs (:184-250), glu_down_input (:435-563), finish_and_reduce (:586-609).
"""

import numpy as np
import pytest

import oracle
from mlxl3_amd import synth

F16 = np.float16


def f16(v):
    return np.asarray(v, np.float32).astype(F16).astype(np.float32)


def dense_moe(x, sel, sc, layer, k, cb, mutant=None):
    gu, gu_suh, gu_svh, down, down_suh, down_svh = layer
    experts, _, n_in = gu_suh.shape
    hidden = gu_svh.shape[-1]
    w_gu = oracle.reconstruct_inner(gu, k, cb, n_in, 2 * experts * hidden).astype(np.float64)
    w_d = oracle.reconstruct_inner(down, k, cb, hidden, experts * n_in).astype(np.float64)
    rows, top_k = sel.shape
    y = np.zeros((rows, n_in), np.float32)
    for r in range(rows):
        acc = np.zeros(n_in, np.float32)
        for t in range(top_k):
            e = int(sel[r, t])
            proj = []
            for p in range(2):
                sp = 1 - p if mutant == "suh_projection" else p
                xin = oracle.h128_staged(f16(x[r].astype(np.float32) * gu_suh[e, sp].astype(np.float32)))
                col = (p * experts + e) * hidden
                if mutant == "up_offset" and p == 1:
                    col = (e + 1) % experts * hidden
                raw = xin.astype(np.float64) @ w_gu[:, col:col + hidden]
                sv = gu_svh[e, p].astype(np.float32)
                proj.append(f16(oracle.h128_f32(f16(raw)) * sv))
            g, u = proj
            if mutant == "swap_glu":
                g, u = u, g
            act = f16((g / (np.float32(1) + np.exp(-g))) * u)
            dsu = down_suh[(e + 1) % experts if mutant == "down_suh_expert" else e]
            din = f16(oracle.h128_f32(f16(act * dsu.astype(np.float32))))
            d = din.astype(np.float64) @ w_d[:, e * n_in:(e + 1) * n_in]
            d = oracle.h128_staged(f16(d))
            if mutant != "no_svh":
                d = f16(d * down_svh[e].astype(np.float32))
            acc += f16(d * np.float32(sc[r, t]))
        y[r] = acc
    return y.astype(F16)


def case(in_f=256, hidden=256, experts=6, top_k=2, rows=5, k=3, seed=3):
    layer = synth.moe_layer(seed, 500, in_f, hidden, experts, k)
    x = synth.activations(seed, 510, rows, in_f)
    sel, sc = synth.moe_routes(seed, 520, rows, experts, top_k)
    return x, sel, sc, layer


def rel_l2(a, b):
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("k,cb", [(2, 0), (3, 0), (3, 1), (4, 2)])
def test_oracle_moe_matches_dense_composition(k, cb):
    x, sel, sc, layer = case(k=k)
    got = oracle.moe_forward(x, sel, sc, *layer, k, cb)
    want = dense_moe(x, sel, sc, layer, k, cb)
    # f32 tile-order vs f64 dense accumulation: rare f16 flips before the glue
    assert rel_l2(got, want) < 1e-3
    rms = np.sqrt(np.mean(want.astype(np.float64) ** 2))
    assert np.abs(got.astype(np.float64) - want).max() < 1e-2 * rms


@pytest.mark.parametrize("mutant", ["swap_glu", "up_offset", "suh_projection", "down_suh_expert",
                                    "no_svh"])
def test_dense_composition_detects_planted_mistakes(mutant):
    x, sel, sc, layer = case()
    got = oracle.moe_forward(x, sel, sc, *layer, 3, 0)
    wrong = dense_moe(x, sel, sc, layer, 3, 0, mutant=mutant)
    assert rel_l2(wrong, got) > 0.05


def test_oracle_moe_scores_scale_exactly():
    x, sel, sc, layer = case()
    y1 = oracle.moe_forward(x, sel, sc, *layer, 3, 0)
    y2 = oracle.moe_forward(x, sel, (sc.astype(np.float32) * 2).astype(F16), *layer, 3, 0)
    np.testing.assert_array_equal(y2, (y1.astype(np.float32) * 2).astype(F16))


def test_oracle_moe_expert_relabelling_is_exact():
    in_f, hidden, experts, k = 256, 128, 5, 2
    x, sel, sc, layer = case(in_f=in_f, hidden=hidden, experts=experts, k=k, rows=6)
    gu, gu_suh, gu_svh, down, down_suh, down_svh = layer
    perm = np.array([3, 0, 4, 1, 2])  # new expert i is old expert perm[i]
    inv = np.argsort(perm)
    ht, it = hidden // 16, in_f // 16
    gate = gu[:, :experts * ht].reshape(gu.shape[0], experts, ht, -1)[:, perm]
    up = gu[:, experts * ht:].reshape(gu.shape[0], experts, ht, -1)[:, perm]
    gu2 = np.concatenate([gate.reshape(gu.shape[0], experts * ht, -1),
                          up.reshape(gu.shape[0], experts * ht, -1)], axis=1)
    down2 = down.reshape(down.shape[0], experts, it, -1)[:, perm].reshape(down.shape)
    layer2 = (gu2, gu_suh[perm], gu_svh[perm], down2, down_suh[perm], down_svh[perm])
    sel2 = inv[sel].astype(np.uint32)
    y1 = oracle.moe_forward(x, sel, sc, *layer, k, 0)
    y2 = oracle.moe_forward(x, sel2, sc, *layer2, k, 0)
    np.testing.assert_array_equal(y1, y2)


def test_oracle_moe_rejects_out_of_bank_routes():
    x, sel, sc, layer = case()
    bad = sel.copy()
    bad[0, 0] = 6
    with pytest.raises(ValueError):
        oracle.moe_forward(x, bad, sc, *layer, 3, 0)


# ---- GELU banks (forward_gelu, moe.rs:1087-1153) ----
# The second composition is built from the linear oracle (engine glue, mode 1:
# expert_mapped is that linear on the expert's tile columns with its scales,
# linear.rs:3125-3137, :3325-3331) and the dense GEGLU, both pinned on their
# own; each slot's output is f16(down * score) and the top-k sum is taken in
# f32 and rounded once, as the SiLU path's finish_and_reduce.


def gelu_composition(x, sel, sc, layer, k, cb, logical, mutant=None):
    gu, gu_suh, gu_svh, down, down_suh, down_svh = layer
    experts, _, n_in = gu_suh.shape
    hidden = gu_svh.shape[-1]
    ht, it = hidden // 16, n_in // 16
    rows, top_k = sel.shape
    y = np.zeros((rows, n_in), np.float32)
    for r in range(rows):
        acc = np.zeros(n_in, np.float32)
        for t in range(top_k):
            e = int(sel[r, t])
            proj = []
            for p in range(2):
                cols = slice((p * experts + e) * ht, (p * experts + e + 1) * ht)
                proj.append(oracle.forward(x[r:r + 1], gu[:, cols], gu_suh[e, p], gu_svh[e, p],
                                           k, cb, mode=1)[0])
            g, u = proj
            if mutant == "swap_glu":
                g, u = u, g
            act = oracle.swiglu(g, u) if mutant == "silu" else oracle.geglu(g, u)
            if mutant != "no_mask":
                act = act.copy()
                act[logical:] = 0
            d = oracle.forward(act[None], down[:, e * it:(e + 1) * it], down_suh[e], down_svh[e],
                               k, cb, mode=1)[0]
            acc += f16(d.astype(np.float32) * np.float32(sc[r, t]))
        y[r] = acc
    return y.astype(F16)


@pytest.mark.parametrize("k,cb,logical", [(3, 0, 200), (2, 1, 256), (4, 2, 96)])
def test_oracle_gelu_moe_matches_linear_composition(k, cb, logical):
    x, sel, sc, layer = case(k=k)
    got = oracle.moe_forward(x, sel, sc, *layer, k, cb, activation="gelu", logical_hidden=logical)
    want = gelu_composition(x, sel, sc, layer, k, cb, logical)
    # the same arithmetic apart from the GEMV's summation order (tile walk vs
    # dense): rare f16 flips before the glue
    assert rel_l2(got, want) < 1e-3
    rms = np.sqrt(np.mean(want.astype(np.float64) ** 2))
    assert np.abs(got.astype(np.float64) - want).max() < 1e-2 * rms


@pytest.mark.parametrize("mutant", ["swap_glu", "silu", "no_mask"])
def test_gelu_composition_detects_planted_mistakes(mutant):
    x, sel, sc, layer = case()
    got = oracle.moe_forward(x, sel, sc, *layer, 3, 0, activation="gelu", logical_hidden=128)
    wrong = gelu_composition(x, sel, sc, layer, 3, 0, 128, mutant=mutant)
    assert rel_l2(wrong, got) > 0.05


def test_oracle_gelu_logical_width_masks_columns():
    # logical_hidden = hidden zeroes nothing (the default); a narrower width
    # changes the output; a bank whose GEGLU outputs past the width are zero
    # anyway (down_suh zero there) cannot tell the two apart
    x, sel, sc, layer = case()
    gu, gu_suh, gu_svh, down, down_suh, down_svh = layer
    full = oracle.moe_forward(x, sel, sc, *layer, 3, 0, activation="gelu")
    same = oracle.moe_forward(x, sel, sc, *layer, 3, 0, activation="gelu", logical_hidden=256)
    np.testing.assert_array_equal(full, same)
    narrow = oracle.moe_forward(x, sel, sc, *layer, 3, 0, activation="gelu", logical_hidden=128)
    assert rel_l2(narrow, full) > 0.05
    dsu = down_suh.copy()
    dsu[:, 128:] = 0
    layer2 = (gu, gu_suh, gu_svh, down, dsu, down_svh)
    a = oracle.moe_forward(x, sel, sc, *layer2, 3, 0, activation="gelu", logical_hidden=128)
    b = oracle.moe_forward(x, sel, sc, *layer2, 3, 0, activation="gelu")
    np.testing.assert_array_equal(a, b)


# ---- the glue steps as ops (swiglu_down_input, finish_and_reduce) ----


def test_oracle_finish_and_reduce_matches_staged_composition():
    # built from the pinned staged Hadamard: f16(f16(H(f16(raw)) * svh) * score),
    # summed in f32 over top-k in slot order and rounded once
    rng = np.random.default_rng(11)
    rows, top_k, width = 4, 3, 256
    raw = (rng.normal(0, 30, (rows * top_k, width))).astype(np.float32)
    svh = rng.uniform(0.5, 1.5, (rows * top_k, width)).astype(F16)
    sc = rng.uniform(0, 1, (rows, top_k)).astype(F16)
    got = oracle.finish_and_reduce(raw, svh, sc)
    v = oracle.h128_staged(f16(raw))
    part = f16(f16(v * svh.astype(np.float32)) * sc.reshape(-1, 1).astype(np.float32))
    want = part.reshape(rows, top_k, width).sum(axis=1, dtype=np.float32).astype(F16)
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


def test_oracle_swiglu_down_input_matches_f32_glue_composition():
    # glu_down_input with SiLU from the pinned f32 Hadamard: numpy's f32 exp may
    # differ from expf in the last bit, so the match is near-total, not exact
    rng = np.random.default_rng(12)
    slots, hidden, experts = 6, 256, 3
    gate_up = rng.normal(0, 40, (slots * 2, hidden)).astype(np.float32)
    gu_svh = (rng.uniform(0.5, 1.5, (experts, 2, hidden)) / 16).astype(F16)
    down_suh = rng.choice([-1.0, 1.0], (experts, hidden)).astype(F16)
    sel = rng.integers(0, experts, slots).astype(np.uint32)
    got = oracle.swiglu_down_input(gate_up, gu_svh, down_suh, sel).astype(np.float32)
    want = np.empty_like(got)
    for s in range(slots):
        e = sel[s]
        g = f16(oracle.h128_f32(f16(gate_up[2 * s])) * gu_svh[e, 0].astype(np.float32))
        u = f16(oracle.h128_f32(f16(gate_up[2 * s + 1])) * gu_svh[e, 1].astype(np.float32))
        act = f16((g / (np.float32(1) + np.exp(-g))) * u)
        want[s] = f16(oracle.h128_f32(f16(act * down_suh[e].astype(np.float32))))
    assert rel_l2(got, want) < 1e-3
    assert np.mean(got == want) > 0.99
