"""The library's host code (argument checks, error strings, the kernel
registry with its descriptor and backend_config parsing, the tile table and
TilePlanner, ExecutionArena, PJRT program parsing, the cblas_sgemm front end)
built with AddressSanitizer and UndefinedBehaviorSanitizer
(tests/cpp/build_sanitize.py) and driven with valid, invalid and extreme
arguments by tests/cpp/host_sanitize.cpp.  CPU only: every call fails its
checks or reaches the HIP runtime, which finds no device here."""
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BINARY = os.path.join(HERE, "cpp", "host_sanitize")


def _binary():
    if not os.path.exists(BINARY):
        sys.path.insert(0, os.path.join(HERE, "cpp"))
        import build_sanitize

        build_sanitize.build()
    return BINARY


def test_host_code_under_asan_ubsan(tmp_path):
    if subprocess.run(["g++", "--version"], capture_output=True).returncode != 0:
        pytest.skip("no g++")
    env = dict(os.environ)
    # the HIP runtime is not instrumented; its allocations are not ours to audit
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env["HIP_VISIBLE_DEVICES"] = ""  # never a device, also where one exists
    r = subprocess.run([_binary()], capture_output=True, text=True, env=env, cwd=tmp_path, timeout=600)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
    assert "0 failed expectations" in r.stdout
