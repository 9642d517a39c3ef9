"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

Builds tests/sanitize/harness.cpp with the host-side descriptor validation
and workspace layout of the attention entry points
(femtochat_amd/csrc/attn_problem.hpp) and the C restatement oracle/fa1.c,
with g++/gcc and -fsanitize=address,undefined (no recovery), and runs it:
every out-of-bounds access, overflow or undefined operation aborts the run.
The harness also checks fa1.c's forward against a float64 softmax attention
on ragged shapes (T not a multiple of its 512-wide blocks).
"""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]


@pytest.mark.skipif(shutil.which("g++") is None or shutil.which("gcc") is None, reason="needs gcc and g++")
def test_host_code_under_sanitizers(tmp_path):
    fa1_o = tmp_path / "fa1.o"
    exe = tmp_path / "harness"
    r = subprocess.run(["gcc", *SAN, "-std=c11", "-c", str(ROOT / "oracle" / "fa1.c"), "-o", str(fa1_o)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run(["g++", *SAN, "-std=c++17", "-Wall", "-Werror", str(ROOT / "tests" / "sanitize" / "harness.cpp"),
                        str(fa1_o), "-o", str(exe), "-lm"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    env = {"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=1", "UBSAN_OPTIONS": "print_stacktrace=1",
           "PATH": "/usr/bin:/bin"}
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("ok"), r.stdout
