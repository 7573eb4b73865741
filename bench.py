"""Benchmark of the EXL3 quantized-linear hot path on one MI355X.

Headline (BASELINE.json metric): effective HBM GB/s of the batch-1 QMV on the
north-star shape (in=4096, out=14336, K=4, 3INST), plus QMM TFLOPS at M=512
on the same shape.  A step is one EXL3 linear forward over one batch.

Protocol:
* weights: one seeded synthetic trellis (mlxl3_amd.synth) replicated into
  ceil(2 GiB / trellis bytes) device copies; consecutive steps rotate over the
  copies so every launch streams its weights from HBM, not from the 256 MB
  Infinity Cache;
* the timed steps run as HIP graph replays on one stream, in --windows (21)
  windows of exactly --steps steps, each bracketed by torch.cuda.synchronize()
  and HIP events recorded on that stream behind a short device spin (so the
  events time the GPU's work, not the CPU's submission); the headline is the
  median window (min / mean / max under "timing"); before each leg's warmup
  steps ~50 ms of untimed replays of the leg's own graph bring the GPU to its
  steady state (short windows would otherwise time the ramp after the setup:
  20-step NS windows read 15.2 us cold against 14.4 us settled on one box);
* value = algorithmic bytes per step / time per step, bytes =
  in*out*K/8 + M*in*2 + M*out*2 + in*2 + out*2 (each tensor once);
* roofline.valu_ceiling: the QMV's measured SQ_INSTS_VALU as an issue-bound
  time (profiles/traffic.json), i.e. how far the decode arithmetic alone keeps
  the kernel from the HBM roofline;
* cpu_baseline: the C oracle (oracle/, decode-at-use GEMV, OpenMP) on this
  host over bounded samples of the headline and of C1, C2 (M 16/128), one C3
  layer, C4 and C5 (M 4/16), with this process's CPU share and one thread;
* ceilings (reference only): this GPU's measured streaming-read bandwidth over
  4 GiB and a dense fp16 GEMM (M=512) / GEMV (M=1) at the same shape through
  torch's library kernels, next to the spec peaks the roofline fractions use.

    python bench.py [--gpus 1] [--steps 2000] [--warmup 200]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 FLOP/clk, dense
ROTATE_BYTES = 2 << 30


def alg_bytes(n_in, n_out, k, rows, bias=False):
    return n_in * n_out * k // 8 + rows * n_in * 2 + rows * n_out * 2 + n_in * 2 + n_out * 2 + (
        n_out * 2 if bias else 0)


def make_rotation(n_in, n_out, k, cb, seed, max_copies=None):
    import numpy as np
    import torch

    import mlxl3_amd
    from mlxl3_amd import synth

    tr, suh, svh, _ = synth.linear_layer(seed, 0, n_in, n_out, k)
    dev = torch.device("cuda")
    base = torch.from_numpy(tr.view(np.int16)).to(dev)
    suh_t = torch.from_numpy(suh).to(dev)
    svh_t = torch.from_numpy(svh).to(dev)
    copies = max(2, math.ceil(ROTATE_BYTES / base.numel() / 2))
    if max_copies:
        copies = max(1, min(copies, max_copies))
    weights = [base] + [base.clone() for _ in range(copies - 1)]
    lins = [mlxl3_amd.Exl3Linear(w, suh_t, svh_t, None, k, cb) for w in weights]
    return lins, weights


def settle(replay, seconds=0.05):
    """Replay the leg's own graph (all rotated copies) for `seconds`, untimed,
    before its warmup steps.  A GPU that has idled or run other work (the
    CPU-side setup between legs) needs tens of milliseconds of this workload to
    reach its steady state: 20-step NS windows read 15.2 us right after other
    work and 14.4 us after 50 ms of the workload on one box (50 ms of dense
    GEMMs instead left the first windows at 15.5-16 us)."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        replay()
        torch.cuda.synchronize()


def time_steps(lins, x, steps, warmup, ws, windows=1):
    """Run warmup steps, then `windows` timed windows of exactly `steps` steps
    each, as graph replays on one stream.  Each window is bracketed by HIP
    events recorded on that stream behind a short device spin, so the CPU has
    queued the whole window before its start event runs and the events time the
    GPU's work only.  Returns (median ms per step over the windows, y,
    per-window ms per step)."""
    import torch

    n = len(lins)
    stream = torch.cuda.current_stream()

    def capture(count):
        g = torch.cuda.CUDAGraph()
        outs = []
        with torch.cuda.graph(g):
            for i in range(count):
                outs.append(lins[i % n].forward(x, workspace=ws))
        return g, outs

    # eager warm-up of every handle (no allocation inside the timed region)
    for lin in lins:
        lin.forward(x, workspace=ws)
    torch.cuda.synchronize()
    full, outs = capture(n)
    parts = {}

    def run(count):
        for _ in range(count // n):
            full.replay()
        if count % n:
            if count % n not in parts:
                parts[count % n] = capture(count % n)[0]
            parts[count % n].replay()

    if steps % n and steps % n not in parts:
        parts[steps % n] = capture(steps % n)[0]  # the window's partial graph, captured untimed
    settle(full.replay)
    run(max(1, warmup))
    torch.cuda.synchronize()
    per = []
    for _ in range(windows):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(200000)  # ~100 us of device spin: the window is queued behind it
        start.record(stream)
        run(steps)
        end.record(stream)
        torch.cuda.synchronize()
        per.append(start.elapsed_time(end) / steps)
    med = sorted(per)[len(per) // 2]
    return med, outs[0], per


def windowed(replay, reps, steps_per_rep, windows):
    """Median ms per step over `windows` windows of `reps` calls of replay()
    (each call `steps_per_rep` steps on the current stream), every window
    bracketed by HIP events behind a short device spin as in time_steps.
    Returns (median ms per step, per-window ms per step)."""
    import torch

    stream = torch.cuda.current_stream()
    settle(replay)
    per = []
    for _ in range(windows):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(200000)
        start.record(stream)
        for _ in range(reps):
            replay()
        end.record(stream)
        torch.cuda.synchronize()
        per.append(start.elapsed_time(end) / (reps * steps_per_rep))
    return sorted(per)[len(per) // 2], per


def window_stats(per):
    """min / mean / max of per-window ms per step, rounded for the JSON line."""
    return {"windows": len(per), "ms_min": round(min(per), 6),
            "ms_mean": round(sum(per) / len(per), 6), "ms_max": round(max(per), 6)}


def _traffic_entry(workload):
    try:
        return json.loads((ROOT / "profiles" / "traffic.json").read_text())[workload]
    except (OSError, KeyError, ValueError):
        return None


def measured_traffic(workload):
    """HBM bytes per step of `workload` (summed over its kernels), as measured
    by rocprofv3 FETCH_SIZE + WRITE_SIZE (scaled by a known-size copy) and
    recorded in profiles/traffic.json; None when not measured."""
    e = _traffic_entry(workload)
    return e.get("hbm_bytes_per_launch") if e else None


def valu_ceiling(workload, ms):
    """The VALU issue bound of the dominant kernel: its measured SQ_INSTS_VALU
    (wave instructions per launch, profiles/traffic.json) x 4 cycles (a wave64
    VALU instruction on a 16-lane SIMD) / 1024 SIMDs / 2.4 GHz, against the
    measured step time; None when not measured."""
    e = _traffic_entry(workload)
    if not e or "valu_insts_per_launch" not in e:
        return None
    us = e["valu_insts_per_launch"] * 4 / (1024 * 2.4e9) * 1e6
    return {"valu_insts": e["valu_insts_per_launch"], "us": round(us, 3),
            "frac": round(us / (ms * 1e3), 4),
            "note": "SQ_INSTS_VALU x 4 cycles / 1024 SIMDs / 2.4 GHz (issue-bound time at peak clock)"}


def cpu_threads():
    """Threads of the CPU legs: this process's CPU share (its affinity mask),
    capped by OMP_NUM_THREADS where the host sets it (the GPU boxes set it to
    their per-GPU share of 16)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def _cpu_time(fn, budget_s, max_calls=1000, warm=False):
    """Seconds per call of fn() (after one untimed call if `warm`), repeated
    until budget_s has passed (at least one timed call)."""
    if warm:
        fn()
    calls, t0 = 0, time.perf_counter()
    while True:
        fn()
        calls += 1
        el = time.perf_counter() - t0
        if el >= budget_s or calls >= max_calls:
            return el / calls, calls


def cpu_baseline(n_in, n_out, k, cb, rows, scale=1.0):
    """The oracle (oracle/: the C restatement of codec.rs + ref/forward.py,
    decode at use, OpenMP) timed on this host over a bounded sample of every
    configuration of the measurement plan, with the GPU legs' algorithmic bytes
    and flops: the headline (in x out, K, rows) at all threads of the process's
    CPU share and at one thread, C1, C2 at M 16 and 128 (both shapes, K 3/4/5),
    one C3 layer (its 7 linears), C4 (the MoE block) and C5 (one layer at M 4
    and 16, K 2 and 4).  `scale` multiplies every leg's time budget."""
    import numpy as np

    import oracle
    from mlxl3_amd import synth

    threads = cpu_threads()
    t_start = time.perf_counter()

    def lin(seed, tid, i, o, kk, c=0):
        return synth.linear_layer(seed, tid, i, o, kk)[:3] + (kk, c)

    def run_lin(L, x, th):
        tr, su, sv, kk, c = L
        return oracle.forward(x, tr, su, sv, kk, c, mode=1, threads=th)

    legs = {}

    def leg(name, fn, budget, nbytes, flops, warm=False, factor=1.0):
        sec, calls = _cpu_time(fn, budget * scale, warm=warm)
        sec *= factor  # a sample of the workload scaled to all of it
        legs[name] = {"ms_per_call": round(sec * 1e3, 3), "calls": calls,
                      "gbs": round(nbytes / sec / 1e9, 3), "gflops": round(flops / sec / 1e9, 3)}
        return sec, calls

    # headline, all threads and one thread (the warm call builds the codebook
    # tables once for every leg)
    L = lin(1, 0, n_in, n_out, k, cb)
    x = synth.activations(1, 0, rows, n_in)
    hb, hf = alg_bytes(n_in, n_out, k, rows), 2.0 * rows * n_in * n_out
    sec, calls = leg("ns", lambda: run_lin(L, x, threads), 5.0, hb, hf, warm=True)
    sec1, calls1 = _cpu_time(lambda: run_lin(L, x, 1), 3.0 * scale)
    del L
    # C1
    L = lin(1, 0, 4096, 4096, 4)
    x1 = synth.activations(1, 0, 1, 4096)
    leg("c1_qmv_4096x4096_k4_m1", lambda: run_lin(L, x1, threads), 1.0,
        alg_bytes(4096, 4096, 4, 1), 2.0 * 4096 * 4096)
    # C2 at M 16 and 128
    for i_, o_ in ((4096, 14336), (14336, 4096)):
        for kk in (3, 4, 5):
            L = lin(2, 0, i_, o_, kk)
            for m in (16, 128):
                xm = synth.activations(2, m, m, i_, outlier_frac=0.01)
                leg(f"c2_{i_}x{o_}_k{kk}_m{m}", lambda: run_lin(L, xm, threads), 0.3,
                    alg_bytes(i_, o_, kk, m), 2.0 * m * i_ * o_)
    del L
    # C3: one dense layer's 7 linears at batch 1
    hid, inter, kv = 4096, 14336, 1024
    c3 = [lin(3, 3000 + 10 * t, i_, o_, 4)
          for t, (i_, o_) in enumerate(((hid, hid), (hid, kv), (hid, kv), (hid, hid),
                                        (hid, inter), (hid, inter), (inter, hid)))]
    xa, xi = synth.activations(3, 1, 1, hid), synth.activations(3, 2, 1, inter)

    def c3_layer():
        for L_ in c3:
            run_lin(L_, xi if L_[0].shape[0] * 16 == inter else xa, threads)

    leg("c3_llama_layer_k4_m1", c3_layer, 2.0,
        sum(alg_bytes(L_[0].shape[0] * 16, L_[0].shape[1] * 16, 4, 1) for L_ in c3),
        sum(2.0 * L_[0].shape[0] * 16 * L_[0].shape[1] * 16 for L_ in c3))
    del c3
    # C4: the MoE block (256 tokens, top-8 of 128 experts, 2048 -> 768, K=3),
    # timed on its first 32 tokens and scaled by 8: the oracle decodes each
    # routed slot's expert tiles at use, so its work is linear in the slots
    ein, eh, E, top, k4, r4, r4s = 2048, 768, 128, 8, 3, 256, 32
    bank = synth.moe_layer(4, 500, ein, eh, E, k4)
    x4 = synth.activations(4, 510, r4, ein)[:r4s]
    sel, sc = synth.moe_routes(4, 520, r4, E, top)
    sel, sc = sel[:r4s], sc[:r4s]
    bank_bytes = (bank[0].size + bank[3].size) * 2
    leg("c4_moe_2048x768_e128_top8_rows256_k3",
        lambda: oracle.moe_forward(x4, sel, sc, *bank, k4, 0, threads=threads), 1.0,
        bank_bytes + r4 * ein * 2 * 2 + (E * 2 * ein + E * 2 * eh + E * eh + E * ein) * 2,
        2.0 * r4 * top * 3 * ein * eh, factor=r4 / r4s)
    legs["c4_moe_2048x768_e128_top8_rows256_k3"]["sample"] = (
        f"first {r4s} of {r4} tokens, time x {r4 // r4s}")
    del bank
    # C5: one 27B-class layer (7 linears, MCG) at M 4 and 16, K 2 and 4
    hid, inter = 5120, 27648
    for kk in (2, 4):
        c5 = [lin(5, 5000 + 10 * t, i_, o_, kk, 1)
              for t, (i_, o_) in enumerate(((hid, hid), (hid, kv), (hid, kv), (hid, hid),
                                            (hid, inter), (hid, inter), (inter, hid)))]
        for m in (4, 16):
            xa5, xi5 = synth.activations(5, m, m, hid), synth.activations(5, 100 + m, m, inter)

            def c5_layer():
                for L_ in c5:
                    run_lin(L_, xi5 if L_[0].shape[0] * 16 == inter else xa5, threads)

            leg(f"c5_layer_mcg_k{kk}_m{m}", c5_layer, 1.0,
                sum(alg_bytes(L_[0].shape[0] * 16, L_[0].shape[1] * 16, kk, m) for L_ in c5),
                sum(2.0 * m * L_[0].shape[0] * 16 * L_[0].shape[1] * 16 for L_ in c5))
        del c5
    wall = time.perf_counter() - t_start
    gbs = hb / sec / 1e9
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "host_cpus": os.cpu_count(),
        "threads_1": {"value": round(hb / sec1 / 1e9, 3), "unit": "GB/s",
                      "ms_per_call": round(sec1 * 1e3, 3), "calls": calls1},
        "sample": (f"the C oracle (engine semantics, decode at use, OpenMP over {threads} "
                   f"threads = this process's CPU share; {os.cpu_count()} CPUs on the host) on "
                   f"the headline linear in={n_in} out={n_out} K={k} rows={rows}: {calls} calls, "
                   f"{sec * 1e3:.2f} ms/call; plus the legs below (each a bounded sample of whole "
                   f"calls, same algorithmic bytes and flops as the GPU legs); {wall:.0f} s in all"),
        "legs": legs,
    }


def moe_leg(steps, warmup, windows=21, rows=256, experts=128):
    """C4 expert block (hidden 2048, `experts` experts x 768, top-8, K=3
    3INST) over `rows` tokens: one SwitchGLU forward per step through the C
    ABI, graph replays rotating over copies of the bank so each step streams
    the experts it routes to from HBM.  rows=256 with 128 experts is C4; 1 and 4
    tokens are the decode shapes (rows < 64: the reference's small-row path);
    16 experts with 256 tokens is one GPU's share of the bank split 8 ways
    (expert parallel).  Bytes per step count each routed expert's weights and
    scales once, plus x and y."""
    import ctypes

    import numpy as np
    import torch

    import mlxl3_amd
    from mlxl3_amd import synth

    in_f, hidden, top_k, k = 2048, 768, 8, 3
    layer = synth.moe_layer(4, 500, in_f, hidden, experts, k)

    def dev(a):
        if a.dtype == np.uint16:
            a = a.view(np.int16)
        elif a.dtype == np.uint32:
            a = a.astype(np.int32)
        return torch.from_numpy(np.ascontiguousarray(a)).cuda()

    bank = [dev(a) for a in layer]
    bank_bytes = (bank[0].numel() + bank[3].numel()) * 2
    copies = max(2, math.ceil(ROTATE_BYTES / bank_bytes))
    trellises = [(bank[0], bank[3])] + [(bank[0].clone(), bank[3].clone()) for _ in range(copies - 1)]
    moes = [mlxl3_amd.Exl3SwitchGlu(g, bank[1], bank[2], d, bank[4], bank[5], top_k=top_k, k=k, cb=0)
            for g, d in trellises]
    x = dev(synth.activations(4, 510, rows, in_f))
    sel_np, sc_np = synth.moe_routes(4, 520, rows, experts, top_k)
    sel, sc = dev(sel_np), dev(sc_np)
    y = torch.empty_like(x)
    lib = mlxl3_amd.load_library()
    nws = int(lib.exl3_moe_workspace_bytes(moes[0]._handle, rows))
    ws = torch.zeros(nws + 4096, dtype=torch.uint8, device="cuda")
    def call(m):  # on the current stream (the capture stream inside torch.cuda.graph)
        rc = lib.exl3_moe_forward(m._handle, x.data_ptr(), 9, rows, sel.data_ptr(), sc.data_ptr(),
                                  9, y.data_ptr(), ws.data_ptr(), ws.numel(),
                                  ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc:
            raise RuntimeError(lib.exl3_last_error().decode())

    for m in moes:
        call(m)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for m in moes:
            call(m)
    reps = max(1, warmup // len(moes))
    for _ in range(reps):
        g.replay()
    torch.cuda.synchronize()
    reps = max(1, math.ceil(steps / len(moes)))
    ms, per = windowed(g.replay, reps, len(moes), windows)
    routed = len(np.unique(sel_np))
    per_expert = bank_bytes // experts + (2 * in_f + 2 * hidden + hidden + in_f) * 2
    nbytes = routed * per_expert + rows * in_f * 2 * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    workload = f"moe_switchglu_{in_f}x{hidden}_e{experts}_top{top_k}_rows{rows}_k{k}_3inst"
    return {
        "workload": workload,
        "ms_per_step": round(ms, 6),
        "steps": reps * len(moes),
        "timing": window_stats(per),
        "bank_copies_rotated": copies,
        "experts_routed": routed,
        "bytes_per_step": nbytes,
        "gflop_per_step": round(2.0 * rows * top_k * 3 * in_f * hidden / 1e9, 3),
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(workload),
        },
    }


def shares_leg(steps, warmup, windows=21):
    """One GPU's share of the multi-GPU layouts (design only beyond one GPU):
    the NS linear column-sharded 8 ways (4096 x 1792, each GPU owns 14 of the
    112 column blocks; x replicated, no exchange) at batch 1, and the C4 expert
    bank split 8 ways by experts (16 experts per GPU) with all 256 tokens x
    top-8 routed to them (what one GPU runs after the all-to-all dispatch).
    Same protocol as the headline and C4 legs."""
    import torch

    from mlxl3_amd import synth

    lins, _w = make_rotation(4096, 1792, 4, 0, seed=2)
    x = torch.from_numpy(synth.activations(2, 0, 1, 4096)).cuda()
    ws = torch.zeros(lins[0].workspace_bytes(1) + 4096, dtype=torch.uint8, device="cuda")
    ms, _, per = time_steps(lins, x, steps, warmup, ws, windows=windows)
    nbytes = alg_bytes(4096, 1792, 4, 1)
    gbs = nbytes / (ms * 1e-3) / 1e9
    col = {"workload": "qmv_4096x1792_k4_3inst_m1 (NS column shard 1/8)",
           "ms_per_step": round(ms, 6), "steps": steps, "timing": window_stats(per),
           "bytes_per_step": nbytes,
           "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None}}
    del lins, _w
    torch.cuda.empty_cache()
    ep = moe_leg(max(8, steps // 40), max(2, warmup // 40), windows=windows, rows=256, experts=16)
    ep["workload"] += " (C4 bank expert-parallel share 1/8)"
    return {"ns_column_shard": col, "moe_expert_share": ep}


def mlp_leg(steps, warmup, rows=1, windows=21):
    """Dense SwiGLU MLP of a decoder layer at the north-star shape (gate/up
    4096 -> 14336, down 14336 -> 4096, K=4 3INST): exl3_mlp_forward (the SwiGLU
    in the gate/up epilogue) against the unfused composition of the reference
    (Exl3Group of gate/up, Array::swiglu, down Exl3Linear), graph replays
    rotating over weight copies so every step streams from HBM."""
    import ctypes

    import torch

    import mlxl3_amd

    in_f, hidden, k = 4096, 14336, 4
    gen = torch.Generator(device="cuda").manual_seed(7)

    def trellis(n_in, n_out):
        return torch.randint(-32768, 32768, (n_in // 16, n_out // 16, 16 * k), dtype=torch.int16,
                             device="cuda", generator=gen)

    def scales(n, fan):
        return ((torch.rand(n, device="cuda", generator=gen) + 0.5) / math.sqrt(fan)).half()

    per_copy = 3 * in_f * hidden * k // 8
    copies = max(2, math.ceil(ROTATE_BYTES / per_copy))
    su_g, su_u, su_d = scales(in_f, 1), scales(in_f, 1), scales(hidden, 1)
    sv_g, sv_u, sv_d = scales(hidden, in_f), scales(hidden, in_f), scales(in_f, hidden)
    layers = []
    for _ in range(copies):
        gate = mlxl3_amd.Exl3Linear(trellis(in_f, hidden), su_g, sv_g, None, k, 0)
        up = mlxl3_amd.Exl3Linear(trellis(in_f, hidden), su_u, sv_u, None, k, 0)
        down = mlxl3_amd.Exl3Linear(trellis(hidden, in_f), su_d, sv_d, None, k, 0)
        layers.append((gate, up, down))
    lib = mlxl3_amd.load_library()
    x = torch.randn(rows, in_f, device="cuda", generator=gen).half()
    y = torch.empty(rows, in_f, dtype=torch.float16, device="cuda")
    g_out = torch.empty(rows, hidden, dtype=torch.float16, device="cuda")
    u_out = torch.empty_like(g_out)
    act = torch.empty_like(g_out)
    gate, up, down = layers[0]
    parts2 = (ctypes.c_void_p * 2)(gate.handle.value, up.handle.value)
    need = max(int(lib.exl3_mlp_workspace_bytes(gate.handle, up.handle, down.handle, rows)),
               int(lib.exl3_group_workspace_bytes(parts2, 2, rows)),
               int(down.workspace_bytes(rows)))
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")

    def check(rc):
        if rc:
            raise RuntimeError(lib.exl3_last_error().decode())

    def fused(layer):
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        g, u, d = layer
        check(lib.exl3_mlp_forward(g.handle, u.handle, d.handle, x.data_ptr(), rows, y.data_ptr(),
                                   ws.data_ptr(), need, s))

    def unfused(layer):
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        g, u, d = layer
        parts = (ctypes.c_void_p * 2)(g.handle.value, u.handle.value)
        outs = (ctypes.c_void_p * 2)(g_out.data_ptr(), u_out.data_ptr())
        check(lib.exl3_group_forward(parts, 2, x.data_ptr(), 9, rows, outs, ws.data_ptr(), need, s))
        check(lib.exl3_swiglu(g_out.data_ptr(), u_out.data_ptr(), act.data_ptr(), rows * hidden, s))
        check(lib.exl3_linear_forward(d.handle, act.data_ptr(), 9, rows, y.data_ptr(), 9,
                                      ws.data_ptr(), need, s))

    def timed(fn):
        for layer in layers:
            fn(layer)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for layer in layers:
                fn(layer)
        for _ in range(max(1, warmup // copies)):
            graph.replay()
        torch.cuda.synchronize()
        reps = max(1, math.ceil(steps / copies))
        ms, _ = windowed(graph.replay, reps, copies, windows)
        return ms, reps * copies

    ms_fused, n = timed(fused)
    y_fused = y.clone()
    ms_unfused, _ = timed(unfused)
    assert torch.equal(y_fused.view(torch.int16), y.view(torch.int16)), "fused != unfused"
    nbytes = per_copy + (2 * in_f + 2 * hidden + hidden + in_f) * 2 + rows * in_f * 2 * 2
    gbs = nbytes / (ms_fused * 1e-3) / 1e9
    flops = 2.0 * rows * 3 * in_f * hidden
    tflops = flops / (ms_fused * 1e-3) / 1e12
    if flops / nbytes >= 315:  # above the ridge point (2516.6 TFLOP/s / 8 TB/s): MFMA-bound
        roof = {"bound": "mfma", "achieved": round(tflops, 2), "peak": FP16_MFMA_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(tflops / FP16_MFMA_PEAK_TFLOPS, 4), "traffic": None}
    else:
        roof = {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None}
    return {
        "workload": f"mlp_swiglu_{in_f}x{hidden}_k{k}_3inst_m{rows}",
        "ms_per_step": round(ms_fused, 6),
        "ms_per_step_unfused": round(ms_unfused, 6),
        "steps": n,
        "weight_copies_rotated": copies,
        "bytes_per_step": nbytes,
        "gflop_per_step": round(flops / 1e9, 3),
        "roofline": roof,
    }


def _dev_linear(n_in, n_out, k, cb, gen, out_scale=1.0):
    """An Exl3Linear over device-generated random trellis words (every bitstream
    is a valid trellis) and +-U(0.5, 1.5) f16 scales (svh times out_scale),
    seeded by `gen`."""
    import torch

    import mlxl3_amd

    tr = torch.randint(-32768, 32768, (n_in // 16, n_out // 16, 16 * k), dtype=torch.int16,
                       device="cuda", generator=gen)

    def scales(n):
        sign = torch.randint(0, 2, (n,), device="cuda", generator=gen).half() * 2 - 1
        return (sign * (torch.rand(n, device="cuda", generator=gen) + 0.5)).half()

    return mlxl3_amd.Exl3Linear(tr, scales(n_in), (scales(n_out) * out_scale).half(), None, k, cb)


def _graph_time(fn, steps, warmup):
    """ms per call of fn() (which launches on the current stream), as graph
    replays bracketed by HIP events."""
    import torch

    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        g.replay()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def _rotated_time(n_in, n_out, k, cb, rows, steps, warmup, gen, x=None):
    """ms per forward of one linear, rotating over weight copies of 2 GiB in
    total so that every launch streams its trellis from HBM."""
    import torch

    per = n_in * n_out * k // 8
    copies = max(2, min(256, math.ceil(ROTATE_BYTES / per)))
    lins = [_dev_linear(n_in, n_out, k, cb, gen) for _ in range(copies)]
    if x is None:
        x = torch.randn(rows, n_in, device="cuda", generator=gen).half()
    ws = torch.zeros(lins[0].workspace_bytes(rows), dtype=torch.uint8, device="cuda")
    y = torch.empty(rows, n_out, dtype=torch.float16, device="cuda")
    import ctypes

    import mlxl3_amd

    lib = mlxl3_amd.load_library()

    def step():
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for lin in lins:
            rc = lib.exl3_linear_forward(lin.handle, x.data_ptr(), 9, rows, y.data_ptr(), 9,
                                         ws.data_ptr(), ws.numel(), s)
            if rc:
                raise RuntimeError(lib.exl3_last_error().decode())

    reps = max(1, math.ceil(steps / copies))
    ms = _graph_time(step, reps, max(1, warmup // copies)) / copies
    del lins
    torch.cuda.empty_cache()
    return ms, reps * copies


def configs_leg(steps, warmup, which=("c1", "c2", "c3", "c5"), c2_k=(3, 4, 5),
                c2_m=(16, 128, 512, 2048), c5_k=(2, 4), c5_m=(4, 8, 16)):
    """The remaining configurations of the measurement plan at one GPU:
    C1 (QMV 4096x4096), the C2 QMM sweep ({4096->14336, 14336->4096} x K{3,4,5}
    x M{16,128,512,2048}, 1 % x20 outlier channels), C3 (32 chained dense
    decoder layers at batch 1) and C5 (27B-class verify block, MCG).  `which`
    and the K / M lists pick a subset (profiling runs)."""
    import torch

    import mlxl3_amd
    from mlxl3_amd import synth

    gen = torch.Generator(device="cuda").manual_seed(3)
    out = {}
    if "c1" in which:
        ms, n = _rotated_time(4096, 4096, 4, 0, 1, steps, warmup, gen)
        b = alg_bytes(4096, 4096, 4, 1)
        out["c1"] = {"workload": "qmv_4096x4096_k4_3inst_m1", "ms_per_step": round(ms, 6),
                     "steps": n, "gbs": round(b / ms / 1e6, 1),
                     "frac_hbm": round(b / ms / 1e6 / HBM_PEAK_GBS, 4)}
    sweep = []
    for n_in, n_out in ((4096, 14336), (14336, 4096)) if "c2" in which else ():
        for k in c2_k:
            for m in c2_m:
                x = torch.from_numpy(synth.activations(2, m, m, n_in, outlier_frac=0.01)).cuda()
                st = max(20, steps // (4 if m <= 128 else 40 if m == 512 else 160))
                ms, n = _rotated_time(n_in, n_out, k, 0, m, st, max(4, warmup // 10), gen, x=x)
                tf = 2.0 * m * n_in * n_out / ms / 1e9
                b = alg_bytes(n_in, n_out, k, m)
                entry = {"in": n_in, "out": n_out, "k": k, "m": m, "ms": round(ms, 6),
                         "tflops": round(tf, 1), "frac_mfma": round(tf / FP16_MFMA_PEAK_TFLOPS, 4),
                         "gbs": round(b / ms / 1e6, 1)}
                if m == 16:
                    entry["frac_hbm"] = round(b / ms / 1e6 / HBM_PEAK_GBS, 4)
                sweep.append(entry)
    if sweep:
        out["c2"] = sweep
    if "c3" in which:
        out["c3"] = _c3_chain(gen, max(3, steps // 200), 2)
    if "c5" in which:
        out["c5"] = _c5_layers(gen, max(10, steps // 40), max(2, warmup // 40), c5_k, c5_m)
    return out


def _c3_chain(gen, steps, warmup):
    """C3: 32 dense decoder layers at batch 1, K=4 3INST, chained as
    a=rms(x); q,k,v=W a; h=x+W_o rms(q); x'=h+mlp(rms(h)) with mlp the fused
    SwiGLU MLP (Exl3Mlp: gate/up with the SwiGLU edge, then down; residual f32,
    rms = f16(v / sqrt(mean v^2 + 1e-6)) in torch), one graph per 32-layer step;
    also the same linears without the glue (frac_hbm_linears_only: the library's
    share of the step).  The gate/up output scales carry 1/sqrt(4096):
    with unit-scale outputs of std ~85 the product g*u would overflow f16."""
    import torch

    import mlxl3_amd

    hid, inter, kv = 4096, 14336, 1024
    layers = []
    for _ in range(32):
        q, kk, v, o = (_dev_linear(hid, n, 4, 0, gen) for n in (hid, kv, kv, hid))
        g, u = (_dev_linear(hid, inter, 4, 0, gen, out_scale=1 / 64) for _ in range(2))
        d = _dev_linear(inter, hid, 4, 0, gen)
        layers.append((mlxl3_amd.Exl3Group([q, kk, v]), o, mlxl3_amd.Exl3Mlp(g, u, d)))
    x0 = torch.randn(1, hid, device="cuda", generator=gen)

    def rms(v):
        v = v.float()
        return (v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + 1e-6)).half()

    state = {}

    def chain():
        x = x0.clone()
        for qkv, o, mlp in layers:
            qq, _, _ = qkv(rms(x))
            h = x + o(rms(qq)).float()
            x = h + mlp(rms(h)).float()
        state["y"] = x

    xh = torch.randn(1, hid, device="cuda", generator=gen).half()

    def linears_only():
        for qkv, o, mlp in layers:
            qkv(xh)
            o(xh)
            mlp(xh)

    ms = _graph_time(chain, steps, warmup)
    ms_lin = _graph_time(linears_only, steps, warmup)
    per_layer = (alg_bytes(hid, hid + 2 * kv, 4, 1) + alg_bytes(hid, hid, 4, 1)
                 + alg_bytes(hid, 2 * inter, 4, 1) + alg_bytes(inter, hid, 4, 1))
    b = 32 * per_layer
    y = state["y"]
    assert torch.isfinite(y).all(), "C3 chain overflowed"
    return {"workload": "c3_llama_layer_x32_k4_3inst_m1", "ms_per_step": round(ms, 5),
            "ms_linears_only": round(ms_lin, 5), "bytes_per_step": b,
            "gbs": round(b / ms / 1e6, 1), "gbs_linears_only": round(b / ms_lin / 1e6, 1),
            "frac_hbm": round(b / ms / 1e6 / HBM_PEAK_GBS, 4),
            "frac_hbm_linears_only": round(b / ms_lin / 1e6 / HBM_PEAK_GBS, 4),
            "out_rms": round(float(y.pow(2).mean().sqrt()), 3)}


def _c5_layers(gen, steps, warmup, ks=(2, 4), m_values=(4, 8, 16)):
    """C5: one 27B-class layer of 7 linears (q/k/v as one group, o, and the
    fused SwiGLU MLP: gate/up as one group whose epilogue applies the SwiGLU and
    the down projection's prologue, then down) at M in {4, 8, 16}, K in {2, 4},
    MCG, rotating over layer copies."""
    import torch

    import mlxl3_amd

    hid, inter, kv = 5120, 27648, 1024
    res = []
    for k in ks:
        per = (hid * (hid + 2 * kv) + hid * hid + 2 * hid * inter + inter * hid) * k // 8
        copies = max(2, math.ceil(ROTATE_BYTES / per))
        layers = []
        for _ in range(copies):
            q, kk, v, o = (_dev_linear(hid, n, k, 1, gen) for n in (hid, kv, kv, hid))
            g, u, d = _dev_linear(hid, inter, k, 1, gen), _dev_linear(hid, inter, k, 1, gen), \
                _dev_linear(inter, hid, k, 1, gen)
            layers.append((mlxl3_amd.Exl3Group([q, kk, v]), o, mlxl3_amd.Exl3Mlp(g, u, d)))
        for m in m_values:
            xh = torch.randn(m, hid, device="cuda", generator=gen).half()

            def step():
                for qkv, o, mlp in layers:
                    qkv(xh)
                    o(xh)
                    mlp(xh)

            reps = max(1, math.ceil(steps / copies))
            ms = _graph_time(step, reps, max(1, warmup)) / copies
            b = (alg_bytes(hid, hid + 2 * kv, k, m) + alg_bytes(hid, hid, k, m)
                 + alg_bytes(hid, 2 * inter, k, m) + alg_bytes(inter, hid, k, m))
            res.append({"k": k, "m": m, "cb": "mcg", "ms_per_layer": round(ms, 6),
                        "gbs": round(b / ms / 1e6, 1), "frac_hbm": round(b / ms / 1e6 / HBM_PEAK_GBS, 4)})
        del layers
        torch.cuda.empty_cache()
    return res


def ceilings_leg(n_in, n_out):
    """Measured ceilings of this GPU, reported next to the spec peaks as
    reference only (library kernels through torch, not this build's code): a
    streaming read of 4 GiB (a reduction), a dense fp16 GEMM at the QMM shape
    (M=512, hipBLASLt) and a dense fp16 GEMV at the batch-1 shape, the latter
    rotating over weight copies that together exceed the 256 MB last-level
    cache so every call streams its weights from HBM."""
    import torch

    def timed(fn, reps):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        b.synchronize()
        return a.elapsed_time(b) / reps  # ms

    big = torch.ones(2 << 30, dtype=torch.float16, device="cuda")  # 4 GiB
    as_i64 = big.view(torch.int64)
    read_ms = min(timed(lambda: big.sum(dtype=torch.float32), 10),
                  timed(lambda: torch.amax(as_i64), 10))  # the faster of two reductions
    read_gbs = big.numel() * 2 / (read_ms * 1e-3) / 1e9
    del big, as_i64
    gen = torch.Generator(device="cuda").manual_seed(11)
    w = torch.randn(n_in, n_out, device="cuda", generator=gen).half()
    xm = torch.randn(512, n_in, device="cuda", generator=gen).half()
    gemm_ms = timed(lambda: torch.matmul(xm, w), 50)
    copies = [w] + [torch.randn(n_in, n_out, device="cuda", generator=gen).half() for _ in range(3)]
    x1 = torch.randn(1, n_in, device="cuda", generator=gen).half()
    state = {"i": 0}

    def gemv():
        state["i"] = (state["i"] + 1) % len(copies)
        torch.matmul(x1, copies[state["i"]])

    gemv_ms = timed(gemv, 200)
    res = {
        "stream_read_gbs": round(read_gbs, 1),
        "fp16_gemm_m512_tflops": round(2.0 * 512 * n_in * n_out / (gemm_ms * 1e-3) / 1e12, 1),
        "fp16_gemv_m1_gbs": round(n_in * n_out * 2 / (gemv_ms * 1e-3) / 1e9, 1),
        "shape": f"{n_in}x{n_out}",
        "source": "torch reduction / hipBLASLt GEMM and GEMV, reference only",
    }
    del w, xm, copies, x1
    torch.cuda.empty_cache()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--windows", type=int, default=21,
                    help="timed windows of `steps` steps each; the headline is their median")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-qmm", action="store_true", help="skip the QMM M=512 leg")
    ap.add_argument("--no-moe", action="store_true", help="skip the MoE SwitchGLU leg")
    ap.add_argument("--no-mlp", action="store_true", help="skip the dense SwiGLU MLP leg")
    ap.add_argument("--no-moe-decode", action="store_true",
                    help="skip the MoE decode legs (1 and 4 tokens x top-8 over the C4 bank)")
    ap.add_argument("--no-shares", action="store_true",
                    help="skip the one-GPU-share legs (NS column shard, 16-expert bank)")
    ap.add_argument("--no-ns", action="store_true", help="skip the headline QMV leg (tuning runs)")
    ap.add_argument("--moe-decode-rows", default="1,4",
                    help="token counts of the MoE decode legs (comma-separated)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the C1/C2-sweep/C3/C5 configuration legs")
    ap.add_argument("--configs-only", default="",
                    help="run only these configuration legs (comma list of c1, c2, c3, c5) and "
                         "print their JSON (profiling runs; no headline)")
    ap.add_argument("--c2-k", default="3,4,5", help="C2 sweep K values (with --configs-only)")
    ap.add_argument("--c2-m", default="16,128,512,2048", help="C2 sweep M values")
    ap.add_argument("--c5-k", default="2,4", help="C5 K values")
    ap.add_argument("--c5-m", default="4,8,16", help="C5 block sizes")
    ap.add_argument("--no-ceilings", action="store_true",
                    help="skip the measured stream-read / fp16 GEMM / GEMV reference ceilings")
    ap.add_argument("--k", type=int, default=4)
    ap.add_argument("--cb", type=int, default=0)
    ap.add_argument("--in-features", type=int, default=4096)
    ap.add_argument("--out-features", type=int, default=14336)
    ap.add_argument("--rows", type=int, default=1)
    ap.add_argument("--calibrate-copy-mb", type=int, default=0,
                    help="first run a device-to-device copy of this many MiB (a known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    ap.add_argument("--copies", type=int, default=0,
                    help="cap on rotated weight copies (0: enough for 2 GiB; 1 keeps weights cache-resident)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build's path runs on a single MI355X "
              "(multi-GPU sharding is design-only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    from mlxl3_amd import synth

    torch.cuda.init()
    if args.calibrate_copy_mb:
        src = torch.ones(args.calibrate_copy_mb << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    n_in, n_out, k, cb, rows = args.in_features, args.out_features, args.k, args.cb, args.rows
    decode_rows = [int(v) for v in args.moe_decode_rows.split(",") if v]
    if args.configs_only:  # profiling runs of configuration legs only
        ints = lambda v: tuple(int(t) for t in v.split(",") if t)  # noqa: E731
        print(json.dumps({"configs": configs_leg(
            args.steps, args.warmup, which=tuple(args.configs_only.split(",")),
            c2_k=ints(args.c2_k), c2_m=ints(args.c2_m), c5_k=ints(args.c5_k),
            c5_m=ints(args.c5_m))}), flush=True)
        return
    if args.no_ns:  # tuning runs of the other legs only (the JSON line then has no headline)
        result = {}
        if not args.no_moe_decode:
            result["moe_decode"] = [moe_leg(max(32, args.steps // 10), max(8, args.warmup // 10),
                                            rows=r) for r in decode_rows]
        if not args.no_shares:
            result["shares"] = shares_leg(args.steps, args.warmup)
        if not args.no_moe:
            result["moe"] = moe_leg(max(8, args.steps // 40), max(2, args.warmup // 40))
        print(json.dumps(result), flush=True)
        return
    lins, _w = make_rotation(n_in, n_out, k, cb, seed=2, max_copies=args.copies or None)
    x = torch.from_numpy(synth.activations(2, 0, rows, n_in)).cuda()
    ws = torch.zeros(max(l.workspace_bytes(max(rows, 512)) for l in lins[:1]) + 4096,
                     dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    ms, _, per = time_steps(lins, x, args.steps, args.warmup, ws, windows=args.windows)
    nbytes = alg_bytes(n_in, n_out, k, rows)
    gbs = nbytes / (ms * 1e-3) / 1e9

    result = {
        "metric": "QMV effective HBM GB/s (% of peak) at 4bpw; QMM TFLOPS (% MFMA peak) at M=512",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded splitmix64 trellis, +-U(0.5,1.5) suh/svh, N(0,1) f16 x)",
        "config": {
            "workload": f"qmv_{n_in}x{n_out}_k{k}_{['3inst', 'mcg', 'mul1'][cb]}_m{rows}",
            "in": n_in, "out": n_out, "k": k, "codebook": cb, "rows": rows,
            "weight_copies_rotated": len(lins), "bytes_per_step": nbytes,
        },
        "timing": dict(window_stats(per), steps_per_window=args.steps,
                       protocol="median over windows of exactly `steps` graph-replayed steps, "
                                "each bracketed by HIP events on the launch stream, after "
                                "~50 ms of untimed replays of the rotation graph (settle) "
                                "and the warmup steps"),
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(f"qmv_{n_in}x{n_out}_k{k}_{['3inst', 'mcg', 'mul1'][cb]}_m{rows}"),
            "valu_ceiling": valu_ceiling(
                f"qmv_{n_in}x{n_out}_k{k}_{['3inst', 'mcg', 'mul1'][cb]}_m{rows}", ms),
        },
    }
    del lins, _w
    torch.cuda.empty_cache()

    if not args.no_qmm:
        m = 512
        qlins, _qw = make_rotation(n_in, n_out, k, cb, seed=2, max_copies=16)
        xq = torch.from_numpy(synth.activations(2, 1, m, n_in, outlier_frac=0.01)).cuda()
        wsq = torch.zeros(qlins[0].workspace_bytes(m) + 4096, dtype=torch.uint8, device="cuda")
        qsteps = max(16, args.steps // 20)
        qms, _, qper = time_steps(qlins, xq, qsteps, max(4, args.warmup // 20), wsq,
                                  windows=args.windows)
        tflops = 2.0 * m * n_in * n_out / (qms * 1e-3) / 1e12
        result["qmm"] = {
            "workload": f"qmm_{n_in}x{n_out}_k{k}_m{m}",
            "tflops": round(tflops, 2),
            "ms_per_step": round(qms, 6),
            "steps": qsteps,
            "timing": window_stats(qper),
            "roofline": {
                "bound": "mfma",
                "achieved": round(tflops, 2),
                "peak": FP16_MFMA_PEAK_TFLOPS,
                "unit": "TFLOP/s",
                "frac": round(tflops / FP16_MFMA_PEAK_TFLOPS, 4),
                "traffic": measured_traffic(f"qmm_{n_in}x{n_out}_k{k}_m{m}"),
            },
        }
        del qlins, _qw

    if not args.no_moe:
        result["moe"] = moe_leg(max(8, args.steps // 40), max(2, args.warmup // 40))
    if not args.no_moe_decode:
        result["moe_decode"] = [moe_leg(max(32, args.steps // 10), max(8, args.warmup // 10), rows=r)
                                for r in decode_rows]
    if not args.no_shares:
        result["shares"] = shares_leg(args.steps, args.warmup)
    if not args.no_mlp:
        result["mlp"] = mlp_leg(max(24, args.steps // 10), max(4, args.warmup // 10), rows=1)
        result["mlp_m512"] = mlp_leg(max(24, args.steps // 40), max(4, args.warmup // 40), rows=512)
    if not args.no_configs:
        result["configs"] = configs_leg(args.steps, args.warmup)
    if not args.no_ceilings:
        result["ceilings"] = ceilings_leg(n_in, n_out)

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(n_in, n_out, k, cb, rows)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
