"""Pins the attention-prologue oracle (oracle/rope_norm.py) on the CPU.

Each check is independent of the oracle's own formula: complex
multiplication for the rotation, the plain norm at position 0, the closed
form of the output RMS, finite differences for the backward, torch's
float32 -> bfloat16 conversion and float32 arithmetic for the rounding modes.
Planted mistakes in a copy of the oracle must each fail one of them.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import rope_norm as R


def _inputs(B=2, T=5, NH=3, D=16, L=64, seed=0):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((B, T, NH, D)).astype(np.float32)
    sin, cos = R.tables(L, D)
    return X, sin, cos


def test_tables_closed_forms():
    sin, cos = R.tables(7, 16)
    assert np.all(sin[0] == 0) and np.all(cos[0] == 1)  # position 0: no rotation
    t = np.arange(7)
    np.testing.assert_allclose(sin[:, 0], np.sin(t), rtol=0, atol=2e-7)  # channel 0: inv_freq 1
    # consecutive inverse frequencies differ by base^(-2/D)
    ang = np.arctan2(sin[1], cos[1]).astype(np.float64)
    np.testing.assert_allclose(ang[1:] / ang[:-1], 1e5 ** (-2 / 16), rtol=1e-6)


def test_rotation_is_complex_multiplication():
    X, sin, cos = _inputs(seed=1)
    pos = np.array([[0, 1, 2, 0, 1], [3, 4, 5, 6, 7]], dtype=np.int32)
    u = R.rotate(X, sin, cos, pos, "f64")
    d = X.shape[-1] // 2
    z = X[..., :d].astype(np.float64) + 1j * X[..., d:].astype(np.float64)
    ang = np.arctan2(sin[pos], cos[pos]).astype(np.float64)[:, :, None, :]
    w = z * np.exp(-1j * ang)
    np.testing.assert_allclose(u[..., :d], w.real, rtol=0, atol=1e-6)
    np.testing.assert_allclose(u[..., d:], w.imag, rtol=0, atol=1e-6)


def test_position_zero_is_the_plain_norm():
    X, sin, cos = _inputs(seed=2)
    pos = np.zeros(X.shape[:2], dtype=np.int32)
    y = R.forward(X, sin, cos, pos, "f64")
    x = X.astype(np.float64)
    ref = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 2.0 ** -23) * 1.2
    np.testing.assert_allclose(y, ref, rtol=1e-12)


def test_output_rms_closed_form():
    # The rotation keeps the sum of squares, so RMS(y) = 1.2 sqrt(ms / (ms + eps)).
    X, sin, cos = _inputs(seed=3)
    X = X * 0.05  # small vectors make eps visible
    y = R.forward(X, sin, cos, None, "f64")
    ms = np.mean(X.astype(np.float64) ** 2, axis=-1)
    np.testing.assert_allclose(np.sqrt(np.mean(y * y, axis=-1)), 1.2 * np.sqrt(ms / (ms + 2.0 ** -23)), rtol=1e-12)


def test_positions_index_the_tables():
    X, sin, cos = _inputs(seed=4)
    pos = np.array([[5, 6, 7, 0, 1], [2, 2, 2, 2, 2]], dtype=np.int32)
    y = R.forward(X, sin, cos, pos, "f64")
    # the same rows with default positions after shifting the tables
    for b in range(2):
        for t in range(5):
            one = R.forward(X[b:b + 1, t:t + 1], sin[pos[b, t]:], cos[pos[b, t]:], None, "f64")
            np.testing.assert_allclose(y[b, t], one[0, 0], rtol=1e-12)
    bad = np.array([[0, 1, 2, 3, 64], [0, 0, 0, 0, -1]], dtype=np.int32)
    yb = R.forward(X, sin, cos, bad, "f64")
    assert np.isnan(yb[0, 4]).all() and np.isnan(yb[1, 4]).all() and np.isfinite(yb[0, :4]).all()


def test_backward_finite_differences():
    X, sin, cos = _inputs(B=1, T=3, NH=2, D=16, seed=5)
    pos = np.array([[3, 9, 1]], dtype=np.int32)
    rng = np.random.default_rng(6)
    dY = rng.standard_normal(X.shape)
    dX = R.backward(dY, X, sin, cos, pos, "f64")
    x0 = X.astype(np.float64)
    h = 1e-6
    num = np.zeros_like(x0)
    for idx in np.ndindex(x0.shape):
        xp, xm = x0.copy(), x0.copy()
        xp[idx] += h
        xm[idx] -= h
        num[idx] = np.sum(dY * (R.forward(xp, sin, cos, pos, "f64") - R.forward(xm, sin, cos, pos, "f64"))) / (2 * h)
    np.testing.assert_allclose(dX, num, rtol=1e-6, atol=1e-8)


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32) * 10,
                        # exact ties: halfway between two bf16 values, both parities
                        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 3.0e38, 1e-40], np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(R.bf16_round(x), ref)


def test_low_precision_modes_against_torch():
    X, sin, cos = _inputs(B=2, T=4, NH=2, D=32, seed=8)
    d = 16
    s = torch.from_numpy(sin[:4])[None, :, None, :]
    c = torch.from_numpy(cos[:4])[None, :, None, :]
    x = torch.from_numpy(X)
    # f32: torch float32 elementwise arithmetic (separately rounded operations)
    u32 = torch.cat([x[..., :d] * c + x[..., d:] * s, x[..., :d] * -s + x[..., d:] * c], -1)
    np.testing.assert_array_equal(R.rotate(X, sin, cos, None, "f32"), u32.numpy())
    # bf16: torch bfloat16 tensors round after every operation
    xb = x.to(torch.bfloat16)
    sb, cb = s.to(torch.bfloat16), c.to(torch.bfloat16)
    ub = torch.cat([xb[..., :d] * cb + xb[..., d:] * sb, xb[..., :d] * -sb + xb[..., d:] * cb], -1)
    Xb = xb.to(torch.float32).numpy()
    np.testing.assert_array_equal(R.rotate(Xb, sin, cos, None, "bf16"), ub.to(torch.float32).numpy())
    # and the bf16 forward stays within bf16 tolerance of the mathematics
    yb = R.forward(Xb, sin, cos, None, "bf16")
    y64 = R.forward(Xb, sin, cos, None, "f64")
    # (the f64 reference uses eps(Float32); bf16 adds eps(BFloat16) = 2^-7 to
    # a mean square near 1, so compare against f64 with that eps)
    u = R.rotate(Xb, sin, cos, None, "f64")
    y64b = u / np.sqrt(np.mean(u * u, -1, keepdims=True) + 2.0 ** -7) * 1.2
    assert np.max(np.abs(yb - y64b)) / np.max(np.abs(y64b)) < 2e-2
    assert not np.allclose(y64, y64b, rtol=1e-4)  # the eps of the element type matters


# ---- planted mistakes: each mutated oracle must fail a check above ----------
def _mutant(kind):
    def fwd(X, sin, cos, positions=None, mode="f64"):
        d = X.shape[-1] // 2
        s, c = R._columns(sin, cos, X.shape[0], X.shape[1], positions)
        x = X.astype(np.float64)
        x1, x2 = x[..., :d], x[..., d:]
        if kind == "sign":
            u = np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], -1)
        elif kind == "halves":
            u = np.concatenate([x2 * c + x1 * s, x2 * -s + x1 * c], -1)
        else:
            u = np.concatenate([x1 * c + x2 * s, x1 * -s + x2 * c], -1)
        eps = 0.0 if kind == "no_eps" else 2.0 ** -23
        if kind == "norm_first":
            xn = x / np.sqrt(np.mean(x * x, -1, keepdims=True) + eps)
            u = np.concatenate([xn[..., :d] * c + xn[..., d:] * s, xn[..., :d] * -s + xn[..., d:] * c], -1)
            return u * 1.2
        return u / np.sqrt(np.mean(u * u, -1, keepdims=True) + eps) * 1.2
    return fwd


@pytest.mark.parametrize("kind", ["sign", "halves", "no_eps"])
def test_planted_mistakes_are_caught(kind):
    X, sin, cos = _inputs(seed=9)
    X = X * 0.01  # mean square ~1e-4: eps(Float32) shifts the norm by ~6e-4
    pos = np.array([[0, 1, 2, 3, 4], [5, 6, 7, 8, 9]], dtype=np.int32)
    bad = _mutant(kind)
    good = R.forward(X, sin, cos, pos, "f64")
    # complex-multiplication pin (sign, halves) or the RMS closed form (eps)
    d = X.shape[-1] // 2
    z = X[..., :d].astype(np.float64) + 1j * X[..., d:].astype(np.float64)
    ang = np.arctan2(sin[pos], cos[pos]).astype(np.float64)[:, :, None, :]
    w = z * np.exp(-1j * ang)
    u_ref = np.concatenate([w.real, w.imag], -1)
    ms = np.mean(X.astype(np.float64) ** 2, axis=-1, keepdims=True)
    y_ref = u_ref / np.sqrt(ms + 2.0 ** -23) * 1.2
    # (float32 tables are orthonormal to ~1e-7)
    np.testing.assert_allclose(good, y_ref, rtol=1e-6, atol=1e-7)
    assert not np.allclose(bad(X, sin, cos, pos), y_ref, rtol=1e-4, atol=1e-6)


def test_rotation_and_norm_commute_in_exact_arithmetic():
    # The rotation keeps every pair's norm, so normalising first gives the
    # same result in exact arithmetic (the rounded modes differ).
    X, sin, cos = _inputs(seed=10)
    np.testing.assert_allclose(_mutant("norm_first")(X, sin, cos), R.forward(X, sin, cos, None, "f64"), rtol=1e-6, atol=1e-7)
