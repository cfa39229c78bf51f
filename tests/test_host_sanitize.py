"""libhxm's host-only arithmetic under AddressSanitizer and
UndefinedBehaviorSanitizer on the CPU: the guards that keep 32-bit offsets
and launch grids in range, the K split, the stream-K layout (every stage of
every tile computed once by the segment walk the kernel runs) and the
tuning-cache entry parser
(hexagon-mlir_amd/csrc/host_logic.h, the code the library itself runs),
driven by tests/sanitize/host_logic_check.cpp with boundary values, a seeded
random sweep against 128-bit restatements, and malformed cache lines."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_host_logic_under_asan_and_ubsan(tmp_path):
    exe = tmp_path / "host_logic_check"
    src = os.path.join(ROOT, "tests", "sanitize", "host_logic_check.cpp")
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
                    "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    "-Wall", "-Werror", src, "-o", str(exe)], check=True, timeout=300)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0 and "host_logic ok" in r.stdout, r.stdout + r.stderr
