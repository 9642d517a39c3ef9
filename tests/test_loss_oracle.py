"""Pins the loss-side oracle (oracle/loss.py) on the CPU.

Independent checks: torch.nn.functional.cross_entropy / embedding and their
autograd gradients in float64 (library routines), central finite
differences, closed forms, and planted mistakes in copies of the oracle that
must fail them.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import loss as L


def _case(N=37, V=53, seed=0, ignore_frac=0.2, base=1):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((N, V)) * 3
    t = rng.integers(0, V, N) + base
    t[rng.random(N) < ignore_frac] = -1
    return x, t


@pytest.mark.parametrize("reduction", ["none", "sum", "mean"])
@pytest.mark.parametrize("base", [0, 1])
def test_cross_entropy_matches_torch(reduction, base):
    x, t = _case(seed=1, base=base)
    got = L.cross_entropy(x, t, -1, reduction, base)
    tt = torch.from_numpy(np.where(t == -1, -1, t - base))
    ref = F.cross_entropy(torch.from_numpy(x), tt, ignore_index=-1, reduction=reduction)
    if reduction == "none":
        ref = torch.where(tt == -1, 0.0, ref)
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("reduction", ["none", "sum", "mean"])
def test_gradient_matches_torch_autograd(reduction):
    x, t = _case(seed=2)
    rng = np.random.default_rng(3)
    xt = torch.from_numpy(x).requires_grad_(True)
    tt = torch.from_numpy(np.where(t == -1, -1, t - 1))
    out = F.cross_entropy(xt, tt, ignore_index=-1, reduction=reduction)
    dy = rng.standard_normal(x.shape[0]) if reduction == "none" else 0.7
    (out * torch.as_tensor(dy, dtype=torch.float64)).sum().backward()
    base_delta = rng.standard_normal(x.shape)
    got = L.cross_entropy_gradient(base_delta, x, t, dy, -1, reduction, 1)
    np.testing.assert_allclose(got - base_delta, xt.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_gradient_finite_differences():
    x, t = _case(N=5, V=7, seed=4, ignore_frac=0.3)
    g = L.cross_entropy_gradient(np.zeros_like(x), x, t, 1.0, -1, "mean", 1)
    h = 1e-6
    num = np.zeros_like(x)
    for idx in np.ndindex(x.shape):
        xp, xm = x.copy(), x.copy()
        xp[idx] += h
        xm[idx] -= h
        num[idx] = (L.cross_entropy(xp, t, -1, "mean", 1) - L.cross_entropy(xm, t, -1, "mean", 1)) / (2 * h)
    np.testing.assert_allclose(g, num, rtol=1e-6, atol=1e-9)


def test_closed_forms():
    # equal logits: every valid token's loss is log V; softmax - onehot sums to 0 per row
    N, V = 9, 31
    x = np.full((N, V), 2.5)
    t = np.arange(N) % V + 1
    np.testing.assert_allclose(L.cross_entropy(x, t, -1, "none"), np.log(V), rtol=1e-14)
    x2, t2 = _case(seed=5)
    g = L.cross_entropy_gradient(np.zeros_like(x2), x2, t2, 1.0, -1, "sum")
    np.testing.assert_allclose(g.sum(axis=1), 0.0, atol=1e-12)
    assert np.all(g[t2 == -1] == 0)
    # shift invariance and stability at large logits
    np.testing.assert_allclose(L.cross_entropy(x2 + 1e4, t2, -1, "none"), L.cross_entropy(x2, t2, -1, "none"),
                               rtol=1e-9, atol=1e-9)


def test_in_order_embedding_gradient():
    # the fixed-order float32 gradient equals the float64 one within float32
    # rounding, skips ids outside the table, and leaves a column that receives
    # only zeros (and a -0 in it) with its bits
    rng = np.random.default_rng(3)
    vocab, N, D = 20, 200, 6
    tok = rng.integers(0, vocab, N)
    tok[:5] = [-1, vocab, 4, 4, 4]
    dy = rng.standard_normal((N, D)).astype(np.float32)
    dy[tok == 11] = 0.0
    delta = rng.standard_normal((vocab, D)).astype(np.float32)
    delta[11, 0] = -0.0
    out = L.embedding_gradient_in_order_f32(delta, dy, tok, base=0)
    keep = (tok >= 0) & (tok < vocab)
    ref = L.embedding_gradient(delta, dy[keep], tok[keep], base=0)
    assert np.allclose(out, ref, rtol=1e-5, atol=1e-5)
    assert np.array_equal(out[11].view(np.uint32), delta[11].view(np.uint32))
    # order matters in float32: a planted reverse order changes some bits
    # when a run's values differ widely in magnitude
    big = np.zeros((3, 1), np.float32)
    rows = np.array([[1e8], [1.0], [-1e8]], np.float32)
    fwd = L.embedding_gradient_in_order_f32(big, rows, np.array([0, 0, 0]), base=0)
    assert fwd[0, 0] == 0.0  # (1e8 + 1) rounds to 1e8, minus 1e8 is 0, in this order


def test_embedding_matches_torch():
    rng = np.random.default_rng(6)
    W = rng.standard_normal((50, 12))
    tok = rng.integers(0, 50, 40)
    tok[:5] = 7  # repeats
    np.testing.assert_array_equal(L.embedding(W, tok + 1, 1), F.embedding(torch.from_numpy(tok), torch.from_numpy(W)).numpy())
    Wt = torch.from_numpy(W).requires_grad_(True)
    dy = rng.standard_normal((40, 12))
    (F.embedding(torch.from_numpy(tok), Wt) * torch.from_numpy(dy)).sum().backward()
    delta = rng.standard_normal(W.shape)
    np.testing.assert_allclose(L.embedding_gradient(delta, dy, tok, 0) - delta, Wt.grad.numpy(), rtol=1e-12, atol=1e-12)


# ---- planted mistakes: each must fail a check above --------------------------
def _ce_off_by_one(logits, targets, ignore_index=-1, reduction="mean", base=1):
    return L.cross_entropy(logits, np.where(np.asarray(targets) == ignore_index, ignore_index, np.asarray(targets) + 1 - (np.asarray(targets) - base == logits.shape[1] - 1) * logits.shape[1]), ignore_index, reduction, base)


def _ce_mean_over_all(logits, targets, ignore_index=-1, reduction="mean", base=1):
    losses = L.cross_entropy(logits, targets, ignore_index, "none", base)
    return float(np.mean(losses))


def _ce_no_max(logits, targets, ignore_index=-1, reduction="mean", base=1):
    x = np.asarray(logits, np.float32)  # float32 without the max shift overflows at large logits
    t, valid = L._valid(targets, ignore_index)
    with np.errstate(over="ignore", invalid="ignore"):
        lse = np.log(np.sum(np.exp(x), axis=-1)).astype(np.float64)
    losses = np.where(valid, lse - x[np.arange(len(t)), np.where(valid, t - base, 0)], 0.0)
    return float(np.sum(losses) / np.sum(valid))


@pytest.mark.parametrize("bad", [_ce_off_by_one, _ce_mean_over_all, _ce_no_max])
def test_planted_mistakes_are_caught(bad):
    x, t = _case(seed=7)
    x = x + 100.0  # large logits: exp overflows in float32 without the shift
    tt = torch.from_numpy(np.where(t == -1, -1, t - 1))
    ref = F.cross_entropy(torch.from_numpy(x), tt, ignore_index=-1, reduction="mean").item()
    assert abs(L.cross_entropy(x, t, -1, "mean") - ref) < 1e-10
    got = bad(x, t)
    assert not (np.isfinite(got) and abs(got - ref) < 1e-6)
