"""Phase probe of the single-row QMV (the batch-1 decode kernel).

Builds a variant of the library with the kernel's phase stamps compiled in
(-DEXL3_QMV_PHASES, into mlxl3_amd/_phases/libexl3_hip.so), runs one linear
through the library's own dispatch (Exl3Linear.forward in graph replays that
rotate over 2 GiB of weight copies, as bench.py times it) and prints, over
every wave of the last launch of each of --reps replays, the distribution of

  start     wave entry, after the launch's first wave entered
  prologue  entry -> loop start (xhat in LDS; the first weight loads issued)
  loop      the weight stream
  exchange  loop end -> split-K counter arrival (partials stored, waits,
            barriers, the counter atomic)
  epilogue  arrival -> outputs stored (the last arriver of each column block)
  end       the launch's first entry -> the wave's last stamp

with the shader clock over the loop and the placement of workgroups and waves
on CUs and SIMDs.

    python mlxl3_amd/phases.py --build          # build the probe library (no GPU)
    python mlxl3_amd/phases.py [--in 4096 --out 14336 --k 4 --reps 5]   # GPU
"""

from __future__ import annotations

import argparse
import math
import os
import sys
from collections import Counter
from pathlib import Path

HERE = Path(__file__).resolve().parent
PROBE_LIB = HERE / "_phases" / "libexl3_hip.so"
WORDS = 8  # kPhaseWords
ROTATE_BYTES = 2 << 30


def build() -> Path:
    sys.path.insert(0, str(HERE.parent))
    from mlxl3_amd import build as lib_build

    return lib_build.build(defines=("EXL3_QMV_PHASES",), lib=PROBE_LIB)


def quantiles(v):
    v = sorted(v)
    if not v:
        return None
    n = len(v)
    return v[0], v[n // 10], v[n // 2], v[9 * n // 10], v[-1]


def run(n_in: int, n_out: int, k: int, cb: int, reps: int, seed: int) -> None:
    os.environ["EXL3_LIB"] = str(PROBE_LIB)  # before the package reads it
    sys.path.insert(0, str(HERE.parent))
    import ctypes

    import numpy as np
    import torch

    import mlxl3_amd
    from mlxl3_amd import synth

    if not PROBE_LIB.exists():
        raise SystemExit(f"{PROBE_LIB} is missing: run `python mlxl3_amd/phases.py --build` first")
    lib = mlxl3_amd.load_library()
    lib.exl3_debug_phase_buffer.restype = ctypes.c_int
    lib.exl3_debug_phase_buffer.argtypes = [ctypes.c_void_p]
    dev = torch.device("cuda")
    tr, suh, svh, _ = synth.linear_layer(seed, 0, n_in, n_out, k)
    base = torch.from_numpy(tr.view(np.int16)).to(dev)
    copies = max(2, math.ceil(ROTATE_BYTES / (base.numel() * 2)))
    weights = [base] + [base.clone() for _ in range(copies - 1)]
    suh_t, svh_t = torch.from_numpy(suh).to(dev), torch.from_numpy(svh).to(dev)
    lins = [mlxl3_amd.Exl3Linear(w, suh_t, svh_t, None, k, cb) for w in weights]
    x = torch.from_numpy(synth.activations(seed, 99, 1, n_in)).to(dev)
    ws = torch.zeros(lins[0].workspace_bytes(1), dtype=torch.uint8, device=dev)
    for lin in lins:
        lin.forward(x, workspace=ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for lin in lins:
            lin.forward(x, workspace=ws)
    # one record per wave of the largest single-row grid (col blocks x in/128
    # splits, up to 8 waves per workgroup)
    slots = (n_out // 128) * (n_in // 128) * 8
    buf = torch.zeros(slots * WORDS, dtype=torch.int64, device=dev)
    for _ in range(20):  # steady state (clocks, caches) before anything is read
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(10):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    us_launch = start.elapsed_time(end) * 1e3 / (10 * copies)

    phase = {name: [] for name in ("start", "prologue", "loop", "exchange", "epilogue", "end")}
    clocks, spans = [], []
    by_xcc = {}  # per XCD: (loop end from the launch's first entry, loop time)
    placement = None
    for rep in range(reps):
        buf.zero_()
        torch.cuda.synchronize()
        assert lib.exl3_debug_phase_buffer(ctypes.c_void_p(buf.data_ptr())) == 0
        graph.replay()  # every launch rewrites its slots: the last launch's stamps remain
        torch.cuda.synchronize()
        assert lib.exl3_debug_phase_buffer(None) == 0
        rec = buf.view(-1, WORDS).cpu().numpy().view(np.uint64)
        rec = rec[rec[:, 0] != 0]
        t00 = int(rec[:, 0].min())
        last_end = 0
        cu_waves, simd_waves = Counter(), Counter()
        for r in rec:
            t = [int(v) for v in r]
            is_last = (t[6] >> 48) & 1
            phase["start"].append((t[0] - t00) * 10)
            phase["prologue"].append((t[1] - t[0]) * 10)
            phase["loop"].append((t[2] - t[1]) * 10)
            phase["exchange"].append((t[3] - t[2]) * 10)
            stop = t[3]
            if is_last and t[7]:
                phase["epilogue"].append((t[7] - t[3]) * 10)
                stop = t[7]
            phase["end"].append((stop - t00) * 10)
            last_end = max(last_end, stop)
            if t[2] > t[1]:
                clocks.append((t[5] - t[4]) / ((t[2] - t[1]) * 10.0))
            hw, xcc = t[6] & 0xFFFFFFFF, (t[6] >> 32) & 0xFF
            by_xcc.setdefault(xcc, []).append(((t[2] - t00) * 10, (t[2] - t[1]) * 10))
            cu = (xcc, (hw >> 13) & 7, (hw >> 12) & 1, (hw >> 8) & 15)
            simd_waves[cu + ((hw >> 4) & 3,)] += 1
            cu_waves[cu] += 1
        spans.append((last_end - t00) * 10 / 1000)
        if placement is None:
            per_cu = Counter(v // 4 for v in cu_waves.values())  # 4 waves per workgroup
            per_simd = Counter(simd_waves.values())
            placement = (len(cu_waves), per_cu, len(simd_waves), per_simd, len(rec))

    print(f"QMV {n_in}x{n_out} K={k} cb={cb} M=1: {us_launch:.2f} us per launch in graph replays "
          f"over {copies} rotated weight copies; stamped launch: first entry -> last stamp "
          f"{sum(spans) / len(spans):.2f} us (mean of {reps})")
    cus, per_cu, simds, per_simd, waves = placement
    print(f"placement: {waves} waves on {cus} CUs ("
          + ", ".join(f"{n} CUs with {w} workgroups" for w, n in sorted(per_cu.items()))
          + f"), {simds} SIMDs ("
          + ", ".join(f"{n} with {w} waves" for w, n in sorted(per_simd.items())) + ")")
    clocks.sort()
    print(f"shader clock over the loop: median {clocks[len(clocks) // 2]:.3f} GHz")
    print()
    print("| phase (ns) | min | p10 | median | p90 | max |")
    print("|---|---|---|---|---|---|")
    for name, v in phase.items():
        q = quantiles(v)
        if q:
            print(f"| {name} | " + " | ".join(f"{int(round(a))}" for a in q) + " |")
    print()
    print("| XCD | waves | loop median (ns) | loop max | loop end median | loop end max |")
    print("|---|---|---|---|---|---|")
    for xcc in sorted(by_xcc):
        ends = sorted(e for e, _ in by_xcc[xcc])
        loops = sorted(d for _, d in by_xcc[xcc])
        print(f"| {xcc} | {len(ends) // reps} | {loops[len(loops) // 2]} | {loops[-1]} | "
              f"{ends[len(ends) // 2]} | {ends[-1]} |")


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--build", action="store_true", help="build the probe library and exit")
    ap.add_argument("--in", dest="n_in", type=int, default=4096)
    ap.add_argument("--out", dest="n_out", type=int, default=14336)
    ap.add_argument("--k", type=int, default=4)
    ap.add_argument("--cb", type=int, default=0)
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--seed", type=int, default=1)
    a = ap.parse_args()
    if a.build:
        build()
        return
    run(a.n_in, a.n_out, a.k, a.cb, a.reps, a.seed)


if __name__ == "__main__":
    main()
