"""Build the gfx950 EXL3 library (mlxl3_amd/libexl3_hip.so) with hipcc.

Each kernel family is its own translation unit; they compile in parallel and
link into one shared object that exports the C ABI of include/exl3_hip.h.

    python -m mlxl3_amd.build            # build (always recompiles)

build(defines=..., lib=...) makes a variant of the library (the phase-probe
build of mlxl3_amd/phases.py) without touching the default one.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libexl3_hip.so"
CODEC = HERE / "exl3_codec"  # the codec JSON-lines driver (links LIB)
SOURCES = ["exl3_api.hip", "exl3_qmv.hip", "exl3_qmm.hip", "exl3_moe.hip", "exl3_mapped.hip",
           "exl3_checkpoint.cpp"]
ARCH = "gfx950"

# -ffp-contract=off: every f32 multiply/add in the glue is rounded separately,
# as the reference's stages are; -packed-fp32-ops off: no v_pk_*_f32;
# -fma-mix-insts off: the backend selects f16(f32(a) * f32(b)) as
# v_fma_mix*(a, b, +0), which turns an exact -0 product into +0 (f16 outputs
# such as f16(+0 * svh) with svh < 0 must keep the sign).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-fma-mix-insts",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the EXL3 library needs ROCm's hipcc")
    return path


def _compile(src: Path, obj: Path, defines=()) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *(f"-D{d}" for d in defines), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in res.stderr.splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = True, defines=(), lib: Path = LIB) -> Path:
    """Compile every translation unit and link `lib` (LIB and the codec driver
    by default; a variant library alone when `lib` is another path); returns
    the library's path."""
    srcs = [CSRC / s for s in SOURCES]
    lib = Path(lib)
    with tempfile.TemporaryDirectory(prefix="exl3_build_") as tmp:
        objs = [Path(tmp) / (s.stem + ".o") for s in srcs]
        jobs = min(len(srcs), max(1, os.cpu_count() or 1))
        with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
            list(pool.map(lambda so: _compile(*so, defines), zip(srcs, objs)))
        tmp_lib = Path(tmp) / LIB.name
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp_lib)]
        cmd += [str(o) for o in objs]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed:\n{res.stderr}")
        lib.parent.mkdir(parents=True, exist_ok=True)
        shutil.copy2(tmp_lib, lib)
        if lib != LIB:
            if verbose:
                print(f"built {lib}")
            return lib
        # the codec driver: host code against the library just built
        tmp_codec = Path(tmp) / CODEC.name
        cmd = [hipcc(), "-O2", "-std=c++17", "-Wall", str(CSRC / "exl3_codec.cpp"), "-o",
               str(tmp_codec), f"-L{HERE}", "-lexl3_hip", "-Wl,-rpath,$ORIGIN"]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"codec driver build failed:\n{res.stderr}")
        shutil.copy2(tmp_codec, CODEC)
    if verbose:
        print(f"built {LIB} and {CODEC}")
    return LIB


if __name__ == "__main__":
    build()
