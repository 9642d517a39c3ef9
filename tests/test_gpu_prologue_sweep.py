"""The attention prologue (rotary embedding + RMS norm x 1.2) over a seeded
sweep of shapes, against oracle/rope_norm.py (the restatement of
src/parameters.jl:409-427 and src/gpt.jl:15-20,53-77,103-106).

test_gpu_prologue.py picks a few shapes per code path; this sweep draws the
number of vectors (batch x tokens x heads, so every tail of the kernels'
per-block vector counts comes up), every head dim the prologue takes, tables
longer than the sequence, positions that restart (documents) or none, both
storage types, and the backward written and added.  The list is drawn once
from a fixed seed.
"""
import numpy as np
import pytest
import torch

from femtochat_amd import attention_prologue, delta_attention_prologue_, rotary_embeddings
from oracle import rope_norm as R
from tests.helpers import rel_err, say
from tests.test_gpu_prologue import _ulp_bf16

pytestmark = pytest.mark.gpu


def _draw(n, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    out = []
    for i in range(n):
        D = int(rng.choice([16, 32, 64, 128]))
        B = int(rng.integers(1, 4))
        T = int(rng.choice([1, 2, 3, 31, 32, 33, 63, 64, 65, 127, 129])) if rng.random() < 0.5 else int(rng.integers(1, 300))
        NH = int(rng.integers(1, 13))
        extra = int(rng.choice([0, 0, 5, 1000]))
        docs = bool(rng.random() < 0.5)
        bf16 = bool(i % 2)
        out.append((B, T, NH, D, extra, docs, bf16, int(rng.integers(0, 1 << 30))))
    return out


CASES = _draw(24, seed=1203)


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c[:7])))
def test_prologue_sweep(gpu, case):
    B, T, NH, D, extra, docs, bf16, seed = case
    say(f"prologue B={B} T={T} NH={NH} D={D} L=T+{extra} docs={docs} bf16={bf16}")
    dtype = torch.bfloat16 if bf16 else torch.float32
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(B, T, NH, D, generator=g).to(dtype)
    sin, cos = rotary_embeddings(T + extra, D)
    pos = None
    if docs:
        rng = np.random.default_rng(seed)
        p = np.zeros((B, T), np.int32)
        for b in range(B):
            t = 0
            while t < T:
                n = int(rng.integers(1, T + 1))
                p[b, t:t + n] = np.arange(min(n, T - t))
                t += n
        pos = p
    Xd = X.to(gpu)
    tabs = (sin.to(gpu), cos.to(gpu))
    posd = None if pos is None else torch.from_numpy(pos).to(gpu)
    mode = "bf16" if bf16 else "f32"

    Y = attention_prologue(Xd, tabs, posd).float().cpu().numpy()
    ref = R.forward(X.float().numpy(), sin.numpy(), cos.numpy(), pos, mode)
    if bf16:
        u = _ulp_bf16(Y, ref)
        assert np.max(u) <= 2.0, f"max difference {np.max(u)} bf16 ulp"
        assert np.mean(u > 0) < 0.01 or Y.size < 2000, f"{np.mean(u > 0):.4f} of the elements differ"
    else:
        np.testing.assert_allclose(Y, ref, rtol=4e-7, atol=1e-7)

    dY = torch.randn(X.shape, generator=g).to(dtype)
    gref = R.backward(dY.float().numpy(), X.float().numpy(), sin.numpy(), cos.numpy(), pos, mode)
    dX = torch.full_like(Xd, float("nan"))
    delta_attention_prologue_(dX, dY.to(gpu), Xd, tabs, posd, accumulate=False)
    tol = 2e-2 if bf16 else 1e-5
    assert rel_err(dX.float().cpu().numpy(), gref) < tol
    base = torch.randn(X.shape, generator=g).to(dtype)
    dX2 = base.to(gpu).clone()
    delta_attention_prologue_(dX2, dY.to(gpu), Xd, tabs, posd, accumulate=True)
    got = dX2.float().cpu().numpy() - base.float().numpy()
    assert rel_err(got, gref) < (4e-2 if bf16 else 1e-5)
