"""Pins the optimizer oracle (oracle/optim.py) on the CPU.

Independent checks: torch.optim.AdamW's update formula in float64, the
closed form of the first AdamW step, float64 pow for Julia's Float32 power,
the two branches of Muon's cautious decay, and for Polar Express the
singular value decomposition (the matrix iteration applies the composed
scalar polynomial to the normalised singular values), its transposition
symmetry, and planted mistakes that must fail.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import optim as O


@pytest.mark.parametrize("t", [1, 2, 3, 4, 7, 10, 100, 1000])
def test_julia_pow(t):
    for x in (0.8, 0.9, 0.95, 0.96, 0.995, 0.999):
        ref = np.float32(np.float64(np.float32(x)) ** t) if t != 3 else np.float32(np.float32(x) ** 3)
        got = O.julia_pow_f32(x, t)
        assert abs(float(got) - float(ref)) <= float(np.spacing(ref)), (x, t)


def test_adamw_matches_torch_formula():
    rng = np.random.default_rng(0)
    n = 1000
    f32 = lambda x: np.asarray(x, np.float32).astype(np.float64)  # the reference's Float32 values
    theta, m0, v0 = f32(rng.standard_normal(n)), f32(rng.standard_normal(n) * 0.1), f32(rng.random(n) * 0.01)
    g = f32(rng.standard_normal(n))
    kw = {k: float(np.float32(x)) for k, x in dict(alpha=0.01, beta1=0.9, beta2=0.95, eps=1e-8, lam=0.1).items()}
    got, m, v = O.adamw_step(theta, g, m0, v0, 5, **kw)
    # torch.optim.AdamW's update in float64 (lr, betas, eps, weight_decay), state after 4 steps
    p = torch.tensor(theta, dtype=torch.float64, requires_grad=True)
    opt = torch.optim.AdamW([p], lr=kw["alpha"], betas=(kw["beta1"], kw["beta2"]), eps=kw["eps"],
                            weight_decay=kw["lam"])
    p.grad = torch.tensor(g)
    opt.state[p] = {"step": torch.tensor(4.0, dtype=torch.float64), "exp_avg": torch.tensor(m0),
                    "exp_avg_sq": torch.tensor(v0)}
    opt.step()
    # torch divides sqrt(v) by sqrt(1 - beta2^t); the reference takes sqrt(v / (1 - beta2^t)): equal in exact arithmetic
    np.testing.assert_allclose(got, p.detach().numpy(), rtol=2e-6, atol=2e-7)
    np.testing.assert_allclose(m, opt.state[p]["exp_avg"].numpy(), rtol=2e-6, atol=1e-8)
    np.testing.assert_allclose(v, opt.state[p]["exp_avg_sq"].numpy(), rtol=2e-6, atol=1e-9)


def test_adamw_first_step_closed_form():
    # t = 1 from zero moments: m_hat = g, v_hat = g^2, so the step is alpha g / (|g| + eps)
    rng = np.random.default_rng(1)
    theta, g = rng.standard_normal(64), rng.standard_normal(64)
    got, _, _ = O.adamw_step(theta, g, np.zeros(64), np.zeros(64), 1, 0.02, 0.8, 0.95, 1e-10, 0.01)
    ref = theta * (1 - 0.02 * 0.01) - 0.02 * np.sign(g)
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-6)


def test_adam_update_and_gradient_scale():
    rng = np.random.default_rng(2)
    Th = rng.standard_normal(50).astype(np.float32)
    m, v = rng.standard_normal(20).astype(np.float32), rng.random(20).astype(np.float32)
    out = O.adam_update(Th, 10, m, v, alpha=0.1, beta=0.5, eta=0.01, lam=0.2, eps=1e-8)
    assert np.array_equal(out[:10], Th[:10]) and np.array_equal(out[30:], Th[30:])
    ref = Th[10:30].astype(np.float64) * (1 - 0.01 * 0.2) - 0.1 * m / (np.sqrt(v / 0.5) + 1e-8)
    np.testing.assert_allclose(out[10:30], ref, rtol=1e-6)
    # the gradient scale N divides the gradient: (2g, N=2) == (g, N=1)
    th, g = rng.standard_normal(30), rng.standard_normal(30)
    a = O.adamw_step(th, 2 * g, np.zeros(30), np.zeros(30), 3, 0.01, 0.9, 0.99, 1e-8, 0.0, grad_scale=2.0)
    b = O.adamw_step(th, g, np.zeros(30), np.zeros(30), 3, 0.01, 0.9, 0.99, 1e-8, 0.0)
    np.testing.assert_allclose(a[0], b[0], rtol=1e-6)


def test_muon_update_branches_and_offsets():
    Th = np.array([1.0, -2.0, 3.0, 0.0, 5.0, -1.0, 7.0, 8.0], np.float32)
    X = np.array([[0.5, 0.5], [-1.0, 2.0]], np.float32)
    out = O.muon_update(Th, X, [1, 5], eta=0.1, lam=0.5)
    # index 1: x*th = -1 < 0 -> only -eta x; index 2: 1.5 >= 0 -> also -eta lam th
    assert np.isclose(out[1], -2.0 - 0.05) and np.isclose(out[2], 3.0 - 0.05 - 0.15)
    assert np.isclose(out[5], -1.0 + 0.1 - 0.05 * -1.0) and np.isclose(out[6], 7.0 - 0.2 - 0.35)
    keep = [0, 3, 4, 7]
    assert np.array_equal(out[keep], Th[keep])
    st = O.gather(np.arange(10.0), [2, 6], 3)
    assert np.array_equal(st, [[2, 3, 4], [6, 7, 8]])
    assert np.array_equal(O.scatter(np.zeros(10), st * 10, [2, 6]), [0, 0, 20, 30, 40, 0, 60, 70, 80, 0])


@pytest.mark.parametrize("shape", [(6, 6), (5, 9), (9, 5)])
def test_polar_express_acts_on_singular_values(shape):
    rng = np.random.default_rng(3)
    G = rng.standard_normal((2,) + shape)
    out = O.polar_express(G)
    for j in range(2):
        U, s, Vt = np.linalg.svd(G[j], full_matrices=False)
        scale = float(np.float32(1.01)) * np.sqrt(np.sum(G[j] ** 2)) + float(np.float32(1e-6))
        ref = (U * O.composed_polynomial(s / scale)) @ Vt
        np.testing.assert_allclose(out[j], ref, rtol=1e-9, atol=1e-11)
    # transposition symmetry
    np.testing.assert_allclose(O.polar_express(np.swapaxes(G, 1, 2)), np.swapaxes(out, 1, 2), rtol=1e-9, atol=1e-11)
    # orthogonalisation: singular values of the output lie near 1 (the polynomial's purpose)
    s_out = np.linalg.svd(out[0], compute_uv=False)
    assert np.all(np.abs(s_out - 1) < 0.35)


@pytest.mark.parametrize("mistake", ["reversed", "no_margin", "cubic_only"])
def test_polar_planted_mistakes(mistake):
    rng = np.random.default_rng(4)
    G = rng.standard_normal((1, 7, 4))
    good = O.polar_express(G)
    if mistake == "reversed":
        bad = O.polar_express(G, coefficients=O.COEFFICIENTS[::-1])
    elif mistake == "no_margin":  # normalise by the Frobenius norm without the 1.01 margin
        X = G[0].T / np.sqrt(np.sum(G[0] ** 2))
        for a, b, c in O.COEFFICIENTS:
            A = X @ X.T
            X = a * X + (b * A + c * A @ A) @ X
        bad = X.T[None]
    else:
        bad = O.polar_express(G, coefficients=[(a, b, 0.0) for a, b, _ in O.COEFFICIENTS])
    U, s, Vt = np.linalg.svd(G[0], full_matrices=False)
    scale = float(np.float32(1.01)) * np.sqrt(np.sum(G[0] ** 2)) + float(np.float32(1e-6))
    ref = (U * O.composed_polynomial(s / scale)) @ Vt
    np.testing.assert_allclose(good[0], ref, rtol=1e-9, atol=1e-11)
    assert not np.allclose(bad[0], ref, rtol=1e-6, atol=1e-8)
