"""GPU parity of the attention prologue (rotary embedding + RMS norm x 1.2)
against oracle/rope_norm.py, through the C ABI (femtochat_amd.prologue).

bf16 storage is compared with the oracle's op-by-op bf16 rounding: equal
except where the float32 sum of squares, summed in another order, moves a
rounding (one bf16 unit in the last place of the normalised value, which
the second rounding after the product by 1.2 can turn into two); fp32 storage with the
float32 oracle to a few float32 units.  The backward is compared with the
float64 gradient at the same rounded rotation.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from femtochat_amd import AttentionPrologueFunction, attention_prologue, delta_attention_prologue_, rotary_embeddings
from femtochat_amd import _lib
from oracle import rope_norm as R

from tests.helpers import rel_err, say

pytestmark = pytest.mark.gpu


def _case(gpu, B, T, NH, D, dtype, positions, L=None, seed=0):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(B, T, NH, D, generator=g).to(dtype)
    L = L or max(T, 8)
    sin, cos = rotary_embeddings(L, D)
    pos = None
    if positions == "docs":
        # documents restart at 0 (lengths 1..T)
        p = np.zeros((B, T), np.int32)
        rng = np.random.default_rng(seed)
        for b in range(B):
            t = 0
            while t < T:
                n = int(rng.integers(1, T + 1))
                p[b, t:t + n] = np.arange(min(n, T - t))
                t += n
        pos = torch.from_numpy(p)
    Xd = X.to(gpu)
    tabs = (sin.to(gpu), cos.to(gpu))
    posd = None if pos is None else pos.to(gpu)
    return X, sin, cos, pos, Xd, tabs, posd


def _ulp_bf16(a, b):
    """|a - b| in bf16 units of the larger magnitude (elementwise)."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    m = np.maximum(np.abs(a), np.abs(b))
    ulp = np.where(m > 0, 2.0 ** (np.floor(np.log2(np.maximum(m, 1e-38))) - 7), 1.0)
    return np.abs(a - b) / ulp


@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("positions", [None, "docs"])
def test_forward_bf16_matches_rounded_oracle(gpu, D, positions):
    X, sin, cos, pos, Xd, tabs, posd = _case(gpu, 2, 37, 3, D, torch.bfloat16, positions, seed=D)
    Y = attention_prologue(Xd, tabs, posd).float().cpu().numpy()
    ref = R.forward(X.float().numpy(), sin.numpy(), cos.numpy(), None if pos is None else pos.numpy(), "bf16")
    u = _ulp_bf16(Y, ref)
    assert np.max(u) <= 2.0, f"max difference {np.max(u)} bf16 ulp"
    assert np.mean(u > 0) < 0.01, f"{np.mean(u > 0):.4f} of the elements differ"
    y64 = R.forward(X.float().numpy(), sin.numpy(), cos.numpy(), None if pos is None else pos.numpy(), "f64")
    # against the mathematics with the bf16 eps folded in: within the bf16 contract
    uu = R.rotate(X.float().numpy(), sin.numpy(), cos.numpy(), None if pos is None else pos.numpy(), "f64")
    y64b = uu / np.sqrt(np.mean(uu * uu, -1, keepdims=True) + 2.0 ** -7) * 1.2
    assert rel_err(Y, y64b) < 2e-2
    assert np.isfinite(y64).all()


@pytest.mark.parametrize("D", [16, 64, 128])
@pytest.mark.parametrize("positions", [None, "docs"])
def test_forward_f32_matches_oracle(gpu, D, positions):
    X, sin, cos, pos, Xd, tabs, posd = _case(gpu, 2, 29, 5, D, torch.float32, positions, seed=100 + D)
    Y = attention_prologue(Xd, tabs, posd).cpu().numpy()
    p = None if pos is None else pos.numpy()
    ref32 = R.forward(X.numpy(), sin.numpy(), cos.numpy(), p, "f32")
    ref64 = R.forward(X.numpy(), sin.numpy(), cos.numpy(), p, "f64")
    np.testing.assert_allclose(Y, ref32, rtol=4e-7, atol=1e-7)
    assert rel_err(Y, ref64) < 1e-6


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("D", [32, 128])
def test_backward_matches_oracle(gpu, dtype, D):
    X, sin, cos, pos, Xd, tabs, posd = _case(gpu, 2, 23, 4, D, dtype, "docs", seed=200 + D)
    g = torch.Generator().manual_seed(7)
    dY = torch.randn(X.shape, generator=g).to(dtype)
    mode = "bf16" if dtype == torch.bfloat16 else "f32"
    ref = R.backward(dY.float().numpy(), X.float().numpy(), sin.numpy(), cos.numpy(), pos.numpy(), mode)
    dX = torch.zeros_like(Xd)
    delta_attention_prologue_(dX, dY.to(gpu), Xd, tabs, posd, accumulate=False)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert rel_err(dX.float().cpu().numpy(), ref) < tol
    # accumulate adds onto what dX holds
    base = torch.randn(X.shape, generator=g).to(dtype)
    dX2 = base.to(gpu).clone()
    delta_attention_prologue_(dX2, dY.to(gpu), Xd, tabs, posd, accumulate=True)
    got = dX2.float().cpu().numpy() - base.float().numpy()
    assert rel_err(got, ref) < (1e-5 if dtype == torch.float32 else 4e-2)


def test_autograd_function_gradient(gpu):
    X, sin, cos, pos, Xd, tabs, posd = _case(gpu, 1, 16, 2, 64, torch.float32, None, seed=3)
    Xg = Xd.clone().requires_grad_(True)
    Y = AttentionPrologueFunction.apply(Xg, tabs[0], tabs[1], None)
    g = torch.randn_like(Y)
    (Y * g).sum().backward()
    ref = R.backward(g.cpu().numpy(), X.numpy(), sin.numpy(), cos.numpy(), None, "f32")
    assert rel_err(Xg.grad.cpu().numpy(), ref) < 1e-5


def test_positions_outside_the_tables_poison_the_vector(gpu):
    X, sin, cos, pos, Xd, tabs, posd = _case(gpu, 1, 6, 2, 32, torch.float32, None, L=8, seed=4)
    bad = torch.tensor([[0, 1, 7, 8, -1, 3]], dtype=torch.int32, device=gpu)
    Y = attention_prologue(Xd, tabs, bad).cpu().numpy()
    assert np.isfinite(Y[0, [0, 1, 2, 5]]).all()
    assert np.isnan(Y[0, [3, 4]]).all()


def test_invalid_arguments_raise(gpu):
    X = torch.zeros(1, 4, 2, 48, device=gpu)
    sin, cos = rotary_embeddings(4, 48, device=gpu)
    with pytest.raises(_lib.AttentionError, match="head_dim"):
        attention_prologue(X, (sin, cos))
    X = torch.zeros(1, 4, 2, 32, device=gpu)
    with pytest.raises(ValueError):
        attention_prologue(X, rotary_embeddings(4, 16, device=gpu))


def test_c3_full_size_properties(gpu):
    # C3's Q and K: every output vector has RMS 1.2 sqrt(ms / (ms + eps))
    # (the rotation keeps norms) to bf16 accuracy, and the first and last
    # batch rows match the rounded oracle.
    B, T, H, Hkv, D = 16, 2048, 10, 5, 128
    sin, cos = rotary_embeddings(T, D)
    tabs = (sin.to(gpu), cos.to(gpu))
    for NH, seed in ((H, 11), (Hkv, 12)):
        say(f"prologue C3 full size: NH={NH} seed={seed}")
        g = torch.Generator(device=gpu).manual_seed(seed)
        Xd = torch.randn(B, T, NH, D, device=gpu, generator=g).to(torch.bfloat16)
        Yd = attention_prologue(Xd, tabs)
        x = Xd.float()
        ms = (x * x).mean(-1)
        rms = (Yd.float() ** 2).mean(-1).sqrt()
        expect = 1.2 * torch.sqrt(ms / (ms + 2.0 ** -7))
        assert float(((rms - expect).abs() / expect).max()) < 1e-2
        for b in (0, B - 1):
            ref = R.forward(Xd[b:b + 1].float().cpu().numpy(), sin.numpy(), cos.numpy(), None, "bf16")
            u = _ulp_bf16(Yd[b:b + 1].float().cpu().numpy(), ref)
            assert np.max(u) <= 2.0 and np.mean(u > 0) < 0.01


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_extreme_magnitudes_take_the_exact_division(gpu, dtype):
    # Vectors whose rotated elements fall below 2^-100, are zero, or whose sum
    # of squares overflows (norm = inf) leave the reciprocal-and-correction
    # quotient for a true division; they must still match the oracle.
    B, T, NH, D = 1, 6, 4, 64
    g = torch.Generator().manual_seed(21)
    X = torch.randn(B, T, NH, D, generator=g)
    X[0, 0, 0, :8] = 1e-33  # both halves of the first pairs tiny
    X[0, 0, 0, 32:40] = -1e-33
    X[0, 1, 1, :] = 0.0
    X[0, 2, 2, 5] = 1e-40  # subnormal element next to normal ones
    X[0, 2, 2, 37] = -1e-40
    X[0, 3, 3, :] = 1e20 if dtype == torch.float32 else 1e30  # the float32 sum of squares overflows
    X[0, 4, 0, :] *= 1e-30
    X = X.to(dtype)
    sin, cos = rotary_embeddings(8, D)
    Y = attention_prologue(X.to(gpu), (sin.to(gpu), cos.to(gpu))).float().cpu().numpy()
    mode = "bf16" if dtype == torch.bfloat16 else "f32"
    with np.errstate(over="ignore"):  # the overflowing sum of squares is the case under test
        ref = R.forward(X.float().numpy(), sin.numpy(), cos.numpy(), None, mode)
    assert np.array_equal(np.isnan(Y), np.isnan(ref)) and not np.isnan(ref).any()
    if dtype == torch.float32:
        np.testing.assert_allclose(Y, ref, rtol=4e-7, atol=1e-44)
    else:
        u = _ulp_bf16(Y, ref)
        assert np.max(u) <= 2.0
    assert np.all(Y[0, 1, 1] == 0) and np.all(Y[0, 3, 3] == 0)
