"""The FunctionDef decoder under AddressSanitizer and UBSan (host only).

program.cpp is built with g++ -fsanitize=address,undefined together with
host stand-ins for the runtime (tests/asan/host_stubs.cpp) and a fuzz
driver (tests/asan/fuzz_program.cpp) that compiles every wire fixture,
truncates each at every length and corrupts them 20000 times. A sanitizer
report fails the run."""
from __future__ import annotations

import glob
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_decoder_under_sanitizers(tmp_path):
    exe = tmp_path / "fuzz_program"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", os.path.join(ROOT, "ml-edsl_amd", "csrc", "program.cpp"),
           os.path.join(ROOT, "tests", "asan", "host_stubs.cpp"),
           os.path.join(ROOT, "tests", "asan", "fuzz_program.cpp"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    fixtures = sorted(glob.glob(os.path.join(ROOT, "tests", "golden", "wire", "*.pb")))
    assert len(fixtures) >= 20
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    res = subprocess.run([str(exe), "20000", *fixtures], capture_output=True, text=True, env=env, timeout=600)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-4000:]
    assert "fuzz ok" in res.stdout
