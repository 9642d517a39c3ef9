"""Builds oracle/liboracle_fa1.so from oracle/fa1.c with gcc (test infrastructure)."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "fa1.c"
OUT = HERE / "liboracle_fa1.so"

# x86-64-v3 (AVX2/FMA) runs on the host CPUs of the GPU boxes; -fopenmp for
# the per-(batch, head) split.  No fast-math: the restatement keeps IEEE fp32.
CFLAGS = ["-O3", "-march=x86-64-v3", "-fopenmp", "-fPIC", "-shared", "-std=c11", "-Wall"]


def build() -> Path:
    tmp = OUT.with_suffix(".so.tmp")
    subprocess.run(["gcc", *CFLAGS, str(SRC), "-o", str(tmp), "-lm"], check=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())
