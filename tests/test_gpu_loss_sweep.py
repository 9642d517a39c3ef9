"""Cross-entropy over a seeded sweep of shapes, against the float64 oracle
(oracle/loss.py, the restatement of src/gpt.jl:175-195 and
src/kernels.jl:8-28).

test_gpu_loss.py names each code path on a few chosen shapes; this sweep
draws token counts and vocabulary sizes on and around the kernels' vector
and block edges (1-5, 15-17, 31-33, 63-65, 255-257, 1023-1025, 4095-4097,
32767-32768), reductions, ignored fractions (none, some, all), logit scales
and shifts, and runs the loss, the gradient (with and without a given
log-sum-exp, added and written) and, where the fused kernel takes the
vocabulary (a multiple of 4 up to 32768), the fused pass.  The list is drawn
once from a fixed seed.
"""
import numpy as np
import pytest
import torch

from femtochat_amd import cross_entropy_, cross_entropy_fused_, cross_entropy_gradient_
from oracle import loss as O
from tests.helpers import rel_err, say

pytestmark = pytest.mark.gpu
TOL = 1e-5

_V_EDGES = [1, 2, 3, 4, 5, 15, 16, 17, 31, 32, 33, 63, 64, 65, 255, 256, 257, 1023, 1024, 1025, 4095, 4096, 4097,
            32767, 32768]
_N_EDGES = [1, 2, 3, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257]


def _draw(n, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    out = []
    for _ in range(n):
        V = int(rng.choice(_V_EDGES)) if rng.random() < 0.7 else int(rng.integers(1, 9000))
        N = int(rng.choice(_N_EDGES)) if rng.random() < 0.6 else int(rng.integers(1, 300))
        reduction = str(rng.choice(["none", "sum", "mean"]))
        ignore = float(rng.choice([0.0, 0.3, 1.0], p=[0.4, 0.5, 0.1]))
        scale = float(rng.choice([0.1, 3.0, 30.0]))
        shift = float(rng.choice([0.0, -50.0, 1e4], p=[0.6, 0.2, 0.2]))
        out.append((N, V, reduction, ignore, scale, shift, int(rng.integers(0, 1 << 30))))
    return out


CASES = _draw(32, seed=1202)


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c[:6])))
def test_cross_entropy_sweep(gpu, case):
    N, V, reduction, ignore, scale, shift, seed = case
    say(f"cross-entropy N={N} V={V} {reduction} ignore={ignore} scale={scale} shift={shift}")
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, V, generator=g) * scale + shift
    t = torch.randint(0, V, (N,), generator=g, dtype=torch.int32)
    t[torch.rand(N, generator=g) < ignore] = -1
    xd, td = x.to(gpu), t.to(gpu)
    xs, ts = x.numpy().astype(np.float64), t.numpy()
    keep = ts != -1

    # fp32 logits near a shift s carry their own rounding, about 2^-24 |s| per
    # operand: the log-sum-exp and x - lse inherit a few of those units, and
    # the probabilities exp(x - lse) that relative error (the reference's
    # fp32 arithmetic has the same).
    ulps = 2.0 ** -21 * abs(shift)  # absolute, on the log-sum-exp, the losses and x - lse
    eps = TOL + ulps  # relative, on the probabilities and so on the gradient
    losses, lse = torch.empty(N, device=gpu), torch.empty(N, device=gpu)
    cross_entropy_(losses, xd, td, -1, reduction, lse=lse)
    torch.cuda.synchronize()
    loss_ref = O.cross_entropy(xs, ts, -1, "none", 0)
    got = losses.cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(loss_ref))
    ok = ~np.isnan(loss_ref)
    assert np.all(np.abs(got[ok] - loss_ref[ok]) <= TOL * np.maximum(1.0, np.abs(loss_ref[ok])) + ulps)
    lse_ref = O.token_lse(xs)
    assert np.all(np.abs(lse.cpu().numpy() - lse_ref) <= TOL * np.maximum(1.0, np.abs(lse_ref) - abs(shift)) + ulps)

    dy = torch.randn(N, generator=g) if reduction == "none" else torch.tensor([0.7])
    dyv = dy.numpy() if reduction == "none" else float(dy)
    gref = O.cross_entropy_gradient(np.zeros((N, V)), xs, ts, dyv, -1, reduction, 0)
    base = torch.randn(N, V, generator=g)
    for given in (None, lse):
        # written
        delta = base.to(gpu)
        cross_entropy_gradient_(delta, xd, td, dy.to(gpu), -1, reduction, lse=given, accumulate=False)
        d = delta.cpu().numpy()
        if keep.any():
            assert rel_err(d[keep], gref[keep]) < eps, "written gradient"
        assert np.array_equal(d[~keep], base.numpy()[~keep]), "ignored rows must stay untouched"
        # added: one fp32 addition onto the buffer's values
        delta = base.to(gpu)
        cross_entropy_gradient_(delta, xd, td, dy.to(gpu), -1, reduction, lse=given)
        d = delta.cpu().numpy()
        ref = base.numpy() + gref
        assert np.all(np.abs(d - ref) <= eps * max(np.max(np.abs(gref)), 1e-30) + 2.0 ** -23 * np.abs(ref)), "added"

    if V % 4 == 0 and V <= 32768:
        for accumulate in (False, True):
            delta = base.to(gpu)
            fl, flse = torch.empty(N, device=gpu), torch.empty(N, device=gpu)
            cross_entropy_fused_(fl, delta, xd, td, dy.to(gpu), -1, reduction, lse=flse, accumulate=accumulate)
            torch.cuda.synchronize()
            got = fl.cpu().numpy()
            assert np.all(np.abs(got[ok] - loss_ref[ok]) <= TOL * np.maximum(1.0, np.abs(loss_ref[ok])) + ulps)
            d = delta.cpu().numpy()
            if accumulate:
                ref = base.numpy() + gref
                assert np.all(np.abs(d - ref) <= eps * max(np.max(np.abs(gref)), 1e-30) + 2.0 ** -23 * np.abs(ref))
            elif keep.any():
                assert rel_err(d[keep], gref[keep]) < eps
            assert np.array_equal(d[~keep], base.numpy()[~keep])
