"""AddressSanitizer + UndefinedBehaviorSanitizer builds of the host C++ that
parses untrusted input: the checkpoint reader (csrc/exl3_checkpoint.cpp with
csrc/exl3_json.hpp) and the codec driver (csrc/exl3_codec.cpp, with the JSON
reader again).  Host code only, compiled by ROCm's clang++ as plain C++ (no
device code), linked against the regular libexl3_hip.so for everything else:

  OUTDIR/libexl3_asan.so  the checkpoint entry points (exl3_checkpoint_*,
                          exl3_linear_load, exl3_moe_load*), instrumented; every
                          other symbol resolves to libexl3_hip.so
  OUTDIR/exl3_codec       the codec driver, instrumented, on libexl3_asan.so

    python -m mlxl3_amd.sanitize OUTDIR

A Python process uses them with the environment of `sanitized_env(OUTDIR)`:
the shared ASan runtime preloaded (it carries the UBSan handlers), leak checks
off (the interpreter's own allocations), every report fatal, EXL3_LIB and
EXL3_CODEC pointing at the instrumented builds.
"""

from __future__ import annotations

import glob
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
CLANG = ROCM / "llvm" / "bin" / "clang++"
FLAGS = ["-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
         "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-shared-libasan",
         "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}", "-Wall", "-Wno-unused-function"]


def asan_runtime() -> Path:
    """clang's shared ASan runtime (libclang_rt.asan-x86_64.so)."""
    found = sorted(glob.glob(str(ROCM / "llvm" / "lib" / "clang" / "*" / "lib" / "linux" /
                                 "libclang_rt.asan-x86_64.so")))
    if not found:
        raise RuntimeError("clang's shared ASan runtime is not installed")
    return Path(found[-1])


def _run(cmd):
    res = subprocess.run([str(c) for c in cmd], capture_output=True, text=True)
    if res.returncode:
        raise RuntimeError(f"sanitizer build failed:\n{' '.join(map(str, cmd))}\n{res.stderr}")


def build(outdir) -> tuple[Path, Path]:
    """Build OUTDIR/libexl3_asan.so and OUTDIR/exl3_codec; returns both paths."""
    out = Path(outdir)
    out.mkdir(parents=True, exist_ok=True)
    if not (HERE / "libexl3_hip.so").exists():
        raise RuntimeError("build libexl3_hip.so first (python -m mlxl3_amd.build)")
    rt = asan_runtime()
    rpath = f"-Wl,-rpath,{out}:{HERE}:{ROCM / 'lib'}:{rt.parent}"
    lib = out / "libexl3_asan.so"
    _run([CLANG, *FLAGS, "-fPIC", "-shared", CSRC / "exl3_checkpoint.cpp", "-o", lib,
          f"-L{HERE}", "-lexl3_hip", f"-L{ROCM / 'lib'}", "-lamdhip64", rpath])
    codec = out / "exl3_codec"
    _run([CLANG, *FLAGS, CSRC / "exl3_codec.cpp", "-o", codec, f"-L{out}", "-lexl3_asan",
          f"-L{HERE}", "-lexl3_hip", f"-L{ROCM / 'lib'}", "-lamdhip64", rpath])
    return lib, codec


def sanitized_env(outdir, base=None) -> dict:
    """The environment of a process that runs on the instrumented builds."""
    out = Path(outdir)
    env = dict(os.environ if base is None else base)
    env.update(
        LD_PRELOAD=str(asan_runtime()),
        ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1",
        UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
        EXL3_LIB=str(out / "libexl3_asan.so"),
        EXL3_CODEC=str(out / "exl3_codec"),
    )
    return env


if __name__ == "__main__":
    if len(sys.argv) != 2:
        sys.exit("usage: python -m mlxl3_amd.sanitize OUTDIR")
    for p in build(sys.argv[1]):
        print(p)
