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

from femtochat_amd import MFMAExact, MFMAFast
from femtochat_amd import workloads as W
from oracle import attention_ref as R
from tests.helpers import TOL, gpu_backward, gpu_forward, rel_err, to_np
from tests.test_gpu_parity import _check_case, _dev, _inputs

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


SWEEP_ACC = _draw_cases(24, seed=715)


@pytest.mark.parametrize("case", SWEEP_ACC, ids=lambda c: "-".join(map(str, c[:9])))
def test_sweep_accumulate(gpu, case):
    """The same draw with the gradients added to random values already in the
    buffers (the reference's default, Δflash_attention₁! adds into dQ, dK,
    dV): the sum must be the overwritten result plus those values, added in
    fp32 and rounded once (bit for bit with fp32 storage)."""
    mode, B, T, H, Hkv, D, window, docs, fp32_io, seed = case
    fast = mode == "fast"
    A = MFMAFast() if fast else MFMAExact()
    positions = None
    if docs:
        positions = W.document_positions(T, B, seed=seed % 100003, mean=max(4, T // 3), sigma=1.0, cap=T)
    pos_d = None if positions is None else torch.from_numpy(positions).to(gpu).contiguous()
    Q, K, V, dO = _inputs(seed % 1000, B, T, H, Hkv, D, fast)
    Qd, Kd, Vd = (_dev(x, fast, gpu) for x in (Q, K, V))
    gd = torch.float32 if (fp32_io or not fast) else torch.bfloat16
    dOd = torch.from_numpy(dO).to(device=gpu, dtype=torch.float32 if (fp32_io or not fast) else torch.bfloat16)
    O, l, m = gpu_forward(A, Qd, Kd, Vd, window, pos_d)
    base = [torch.randn(x.shape, device=gpu).to(gd) for x in (Qd, Kd, Vd)]
    fresh = gpu_backward(A, dOd, Qd, Kd, Vd, O, l, m, window, pos_d, grad_dtype=gd)
    added = gpu_backward(A, dOd, Qd, Kd, Vd, O, l, m, window, pos_d, grad_dtype=gd, accumulate=True, init=base)
    torch.cuda.synchronize()
    g_ref = R.backward(dO, Q, K, V, to_np(O), to_np(l), to_np(m), window, positions, fast=fast)
    for name, f, s, b0, r in zip(("dQ", "dK", "dV"), fresh, added, base, g_ref):
        e = rel_err(to_np(f), r)
        assert e <= TOL[mode], f"{name} rel err {e}"
        want = to_np(f) + to_np(b0)
        if gd == torch.float32:
            assert np.array_equal(to_np(s), want), f"{name}: accumulated fp32 differs from fresh + base"
        else:
            assert rel_err(to_np(s), want) <= 1e-2, f"{name}: accumulated bf16"
