"""GPU parity over a seeded sweep of shapes, windows, documents and storage
types, against the float64 oracle (oracle/attention_ref.py, the restatement
of src/kernels.jl:30-96,131-379).

The hand-picked cases in test_gpu_parity.py name each code path; this sweep
draws the parameters instead, so combinations nobody picked also run: T on
and around the tile edges (32, 64, 128 queries or keys) and in between, every
head dim the library takes (D % 16 == 0 up to 128, the non-compiled widths
through zero-padded copies), GQA ratios 1-4, causal, sliding, two-sided and
right-of-query windows (some leaving rows empty), packed documents, and fp32
O/dO/gradients in fast mode.  The list is drawn once from a fixed seed, so
every run checks the same cases and a failure names its parameters.
"""
import numpy as np
import pytest
import torch

from femtochat_amd import workloads as W
from tests.test_gpu_parity import _check_case

pytestmark = pytest.mark.gpu

_EDGES = [1, 2, 31, 32, 33, 63, 64, 65, 96, 127, 128, 129, 191, 255, 256, 257, 383, 511, 513]


def _draw_cases(n: int, seed: int):
    rng = np.random.Generator(np.random.PCG64(seed))
    cases = []
    for i in range(n):
        mode = "fast" if i % 3 else "exact"
        T = int(rng.choice(_EDGES)) if rng.random() < 0.5 else int(rng.integers(3, 600))
        B = int(rng.integers(1, 4))
        D = int(rng.choice([16, 32, 48, 64, 80, 96, 112, 128]))
        Hkv = int(rng.integers(1, 4))
        group = int(rng.integers(1, 5))
        kind = int(rng.integers(0, 5))
        if kind == 0:
            window = (-1, 0)  # causal
        elif kind == 1:
            window = (int(rng.integers(0, T + 1)), 0)  # sliding, left only
        elif kind == 2:
            window = (int(rng.integers(-1, T + 1)), int(rng.integers(1, T + 1)))  # two-sided
        elif kind == 3:
            a = int(rng.integers(1, T + 2))
            window = (-a, a - 1 + int(rng.integers(0, 40)))  # right of the query (empty when right < a)
        else:
            window = (int(rng.integers(0, T + 1)), int(rng.integers(0, 8)))
        docs = bool(rng.random() < 0.3)
        fp32_io = mode == "fast" and bool(rng.random() < 0.25)
        cases.append((mode, B, T, Hkv * group, Hkv, D, window, docs, fp32_io, int(rng.integers(0, 1 << 30))))
    return cases


SWEEP = _draw_cases(48, seed=20261202)


@pytest.mark.parametrize("case", SWEEP, ids=lambda c: "-".join(map(str, c[:9])))
def test_sweep(gpu, case):
    mode, B, T, H, Hkv, D, window, docs, fp32_io, seed = case
    positions = None
    if docs:
        positions = W.document_positions(T, B, seed=seed % 100003, mean=max(4, T // 3), sigma=1.0, cap=T)
    f32 = torch.float32 if fp32_io else None
    _check_case(gpu, mode, B, T, H, Hkv, D, window, positions=positions, seed=seed % 1000, out_dtype=f32,
                grad_dtype=f32, dout_dtype=f32)
