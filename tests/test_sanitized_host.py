"""The host code that reads untrusted input -- the checkpoint reader
(exl3_checkpoint.cpp, exl3_json.hpp) and the codec driver (exl3_codec.cpp) --
built with AddressSanitizer and UndefinedBehaviorSanitizer
(mlxl3_amd/sanitize.py), with the CPU tests of test_checkpoint.py and
test_codec_cli.py run against those builds in a child process: every report is
fatal, so a green run means no memory error or undefined behaviour on any of
their malformed headers, shards, indexes and requests.  The reference runs its
sanitizers in CI the same way (.github/workflows/rust.yml:145-155)."""

import subprocess
import sys
from pathlib import Path

import pytest

from mlxl3_amd import sanitize

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def asan_build(tmp_path_factory):
    try:
        sanitize.asan_runtime()
    except RuntimeError as e:
        pytest.skip(str(e))
    out = tmp_path_factory.mktemp("asan")
    sanitize.build(out)
    return out


def test_instrumented_builds_are_the_ones_loaded(asan_build):
    code = (
        "import ctypes, mlxl3_amd\n"
        "L = mlxl3_amd.load_library()\n"
        "class Info(ctypes.Structure):\n"
        "    _fields_ = [('fname', ctypes.c_char_p), ('fbase', ctypes.c_void_p),\n"
        "                ('sname', ctypes.c_char_p), ('saddr', ctypes.c_void_p)]\n"
        "dl = ctypes.CDLL('libdl.so.2')\n"
        "for name in ('exl3_checkpoint_open', 'exl3_linear_create'):\n"
        "    info = Info()\n"
        "    addr = ctypes.cast(getattr(L, name), ctypes.c_void_p)\n"
        "    assert dl.dladdr(addr, ctypes.byref(info))\n"
        "    print(name, info.fname.decode())\n"
    )
    res = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True,
                         env=sanitize.sanitized_env(asan_build), timeout=300)
    assert res.returncode == 0, res.stderr[-3000:]
    where = dict(line.split() for line in res.stdout.splitlines())
    assert where["exl3_checkpoint_open"].endswith("libexl3_asan.so")
    assert where["exl3_linear_create"].endswith("libexl3_hip.so")


def test_checkpoint_and_codec_tests_under_asan_ubsan(asan_build):
    res = subprocess.run(
        [sys.executable, "-m", "pytest", "tests/test_checkpoint.py", "tests/test_codec_cli.py",
         "-q", "-m", "not gpu", "-p", "no:cacheprovider"],
        cwd=ROOT, capture_output=True, text=True, env=sanitize.sanitized_env(asan_build),
        timeout=600)
    print(res.stdout[-2000:], res.stderr[-4000:])
    assert res.returncode == 0
    assert " passed" in res.stdout and "failed" not in res.stdout
