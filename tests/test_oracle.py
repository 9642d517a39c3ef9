"""Pins the oracle (CPU only).

The reference ships no tests or golden vectors, so every oracle function is
pinned here by checks that a plausible mistake (a dropped scale, a wrong sign,
a transposed operand, an off-by-one window, a wrong GQA head map) fails:

* torch autograd through an independent formulation (explicit masked softmax
  and matmuls, float64) and torch's scaled_dot_product_attention (bool mask,
  enable_gqa) for O and the gradients;
* central finite differences of sum(dO . O) on the README toy config (C1);
* the float32 FA-1 restatement (oracle/fa1.c) against the float64 oracle;
* closed forms and invariants: T=1, single visible key, causal sentinel,
  V scaling, softmax normalisation, GQA == repeated K/V, document mask ==
  per-segment attention, batch/head permutation;
* the committed golden fixtures (tests/golden/c1_golden.npz and the
  document-masked C3 slice, slice_golden.npz);
* the scale identity <dQ, Q> = <dK, K> per (batch, KV group) that the
  full-size GPU tests check (Q -> aQ, K -> K/a leaves the output unchanged);
* the fast-mode rounding variant of the backward (P and dS rounded to bf16):
  its rounding against torch's bfloat16 conversion, and exact agreement with
  the unrounded backward on inputs whose P and dS are bf16 values.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from femtochat_amd import workloads as W
from oracle import attention_ref as R
from oracle import fa1
from oracle import fa1_blas

GOLDEN = Path(__file__).resolve().parent / "golden" / "c1_golden.npz"
SLICE_GOLDEN = Path(__file__).resolve().parent / "golden" / "slice_golden.npz"


def rand(seed, B, T, H, Hkv, D):
    rng = np.random.Generator(np.random.PCG64(seed))
    return (rng.standard_normal((B, T, H, D)), rng.standard_normal((B, T, Hkv, D)),
            rng.standard_normal((B, T, Hkv, D)), rng.standard_normal((B, T, H, D)))


def torch_reference(Q, K, V, dO, window, positions=None):
    """Independent float64 formulation: masked softmax + matmul, gradients by autograd."""
    Qt, Kt, Vt = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (Q, K, V))
    B, T, H, D = Q.shape
    G = H // K.shape[2]
    Kr = Kt.repeat_interleave(G, dim=2)
    Vr = Vt.repeat_interleave(G, dim=2)
    S = torch.einsum("bqhd,bkhd->bhqk", Qt, Kr) / np.sqrt(D)
    q = torch.arange(T)[:, None]
    k = torch.arange(T)[None, :]
    left, right = window
    vis = (k <= q) if (left, right) == (-1, 0) else ((q - left <= k) & (k <= q + right))
    vis = vis[None, None].expand(B, 1, T, T)
    if positions is not None:
        pos = torch.tensor(positions, dtype=torch.int64)
        vis = vis & (k[None, None] >= (q[None, None] - pos[:, None, :, None]))
    S = S.masked_fill(~vis, float("-inf"))
    P = torch.softmax(S, dim=-1)
    O = torch.einsum("bhqk,bkhd->bqhd", P, Vr)
    O.backward(torch.tensor(dO, dtype=torch.float64))
    return O.detach().numpy(), Qt.grad.numpy(), Kt.grad.numpy(), Vt.grad.numpy()


def max_rel(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


CASES = [
    (1, 2, 9, 4, 2, 16, (-1, 0), None),
    (2, 1, 33, 6, 3, 32, (5, 0), None),
    (3, 2, 20, 2, 2, 16, (3, 2), None),
    (4, 1, 40, 4, 1, 16, (-1, 0), "docs"),
    (5, 1, 17, 2, 1, 16, (17, 0), None),
]


def _positions(case_seed, B, T):
    return W.document_positions(T, B, seed=case_seed, mean=6, sigma=0.8, cap=20)


@pytest.mark.parametrize("case", CASES, ids=[str(c[0]) for c in CASES])
def test_oracle_matches_torch_autograd(case):
    seed, B, T, H, Hkv, D, window, pos_kind = case
    Q, K, V, dO = rand(seed, B, T, H, Hkv, D)
    pos = _positions(seed, B, T) if pos_kind else None
    O, l, m = R.forward(Q, K, V, window, pos)
    dQ, dK, dV = R.backward(dO, Q, K, V, O, l, m, window, pos)
    O_t, dQ_t, dK_t, dV_t = torch_reference(Q, K, V, dO, window, pos)
    assert max_rel(O, O_t) < 1e-12
    assert max_rel(dQ, dQ_t) < 1e-10
    assert max_rel(dK, dK_t) < 1e-10
    assert max_rel(dV, dV_t) < 1e-10


def test_oracle_matches_sdpa_gqa():
    B, T, H, Hkv, D = 2, 24, 6, 2, 32
    Q, K, V, dO = rand(11, B, T, H, Hkv, D)
    O, l, m = R.forward(Q, K, V, (-1, 0))
    dQ, dK, dV = R.backward(dO, Q, K, V, O, l, m, (-1, 0))
    Qt, Kt, Vt = (torch.tensor(x, dtype=torch.float64).transpose(1, 2).requires_grad_(True) for x in (Q, K, V))
    Ot = torch.nn.functional.scaled_dot_product_attention(Qt, Kt, Vt, is_causal=True, enable_gqa=True)
    Ot.backward(torch.tensor(dO, dtype=torch.float64).transpose(1, 2))
    assert max_rel(O, Ot.transpose(1, 2).detach().numpy()) < 1e-12
    for g, t in ((dQ, Qt), (dK, Kt), (dV, Vt)):
        assert max_rel(g, t.grad.transpose(1, 2).numpy()) < 1e-10


def test_statistics_closed_form():
    """m = max visible scaled score, l = sum exp(S - m), LSE = logsumexp."""
    B, T, H, Hkv, D = 1, 13, 2, 1, 16
    Q, K, V, _ = rand(21, B, T, H, Hkv, D)
    O, l, m = R.forward(Q, K, V, (4, 1))
    vis = R.visible(T, (4, 1))
    for h in range(H):
        S = Q[0, :, h] @ K[0, :, 0].T / 4.0
        for q in range(T):
            s = S[q][vis[q]]
            assert np.isclose(m[0, h, q], s.max(), rtol=0, atol=1e-14)
            assert np.isclose(l[0, h, q], np.exp(s - s.max()).sum(), rtol=1e-14)
            assert np.isclose(R.lse(l, m)[0, h, q], np.log(np.exp(s).sum()), rtol=1e-13)


def test_single_key_and_T1():
    B, T, H, Hkv, D = 1, 7, 2, 1, 16
    Q, K, V, dO = rand(31, B, T, H, Hkv, D)
    O, l, m = R.forward(Q, K, V, (0, 0))  # every query sees only itself
    assert np.allclose(O, np.repeat(V, H, axis=2), atol=1e-14)
    assert np.allclose(l, 1.0)
    dQ, dK, dV = R.backward(dO, Q, K, V, O, l, m, (0, 0))
    assert np.max(np.abs(dQ)) < 1e-12
    assert np.allclose(dV[:, :, 0], dO.sum(axis=2), atol=1e-12)
    O1, l1, m1 = R.forward(Q[:, :1], K[:, :1], V[:, :1], (-1, 0))
    assert np.allclose(O1, np.repeat(V[:, :1], H, axis=2))
    S = np.einsum("bhd,bd->bh", Q[:, 0], K[:, 0, 0]) / 4.0
    assert np.allclose(m1[:, :, 0], S)


def test_empty_rows():
    Q, K, V, dO = rand(41, 1, 6, 2, 2, 16)
    O, l, m = R.forward(Q, K, V, (-1, 3))  # keys q+1..q+3: the last query sees none
    assert l[0, 0, -1] == 0 and m[0, 0, -1] == -R.FLT_MAX and np.all(O[0, -1] == 0)
    dQ, dK, dV = R.backward(dO, Q, K, V, O, l, m, (-1, 3))
    assert np.all(dQ[0, -1] == 0)


def test_causal_sentinel_equivalence_and_linearity():
    Q, K, V, dO = rand(51, 2, 12, 2, 1, 16)
    a = R.forward(Q, K, V, (-1, 0))
    for w in ((11, 0), (12, 0), (1000, 0)):
        b = R.forward(Q, K, V, w)
        for x, y in zip(a, b):
            assert np.allclose(x, y, rtol=0, atol=0)
    c = R.forward(Q, K, 3.0 * V, (-1, 0))
    assert np.allclose(c[0], 3.0 * a[0], rtol=1e-13)


def test_gqa_equals_repeated_kv_and_permutation():
    B, T, H, Hkv, D = 2, 10, 6, 2, 16
    Q, K, V, dO = rand(61, B, T, H, Hkv, D)
    G = H // Hkv
    O, l, m = R.forward(Q, K, V, (-1, 0))
    Or, lr, mr = R.forward(Q, np.repeat(K, G, 2), np.repeat(V, G, 2), (-1, 0))
    assert np.allclose(O, Or, atol=1e-14)
    g = R.backward(dO, Q, K, V, O, l, m, (-1, 0))
    gr = R.backward(dO, Q, np.repeat(K, G, 2), np.repeat(V, G, 2), Or, lr, mr, (-1, 0))
    assert np.allclose(g[0], gr[0], atol=1e-13)
    assert np.allclose(g[1], gr[1].reshape(B, T, Hkv, G, D).sum(3), atol=1e-13)
    # Batch permutation equivariance.
    p = [1, 0]
    Op, _, _ = R.forward(Q[p], K[p], V[p], (-1, 0))
    assert np.allclose(Op, O[p], atol=1e-14)


@pytest.mark.parametrize("case", CASES, ids=[str(c[0]) for c in CASES])
def test_backward_sum_identities(case):
    # The whole-output identities the full-size GPU tests check: each query's
    # probabilities sum to one over its visible keys and its dS row to zero,
    # so per (batch, KV head) sum_t dV = the group's sum_t dO and sum_t dK = 0.
    # A planted mistake (one key block's dV and dK dropped) must break both.
    seed, B, T, H, Hkv, D, window, pos_kind = case
    Q, K, V, dO = rand(seed, B, T, H, Hkv, D)
    pos = _positions(seed, B, T) if pos_kind == "docs" else None
    O, l, m = R.forward(Q, K, V, window, pos)
    dQ, dK, dV = R.backward(dO, Q, K, V, O, l, m, window, pos)
    G = H // Hkv
    dO_sum = dO.reshape(B, T, Hkv, G, D).sum(axis=(1, 3))
    assert np.allclose(dV.sum(axis=1), dO_sum, atol=1e-12 * np.abs(dO).sum())
    assert np.all(np.abs(dK.sum(axis=1)) <= 1e-12 * np.abs(dK).sum(axis=1) + 1e-300)
    dV_bad, dK_bad = dV.copy(), dK.copy()
    dV_bad[:, :4] = 0.0
    dK_bad[:, :4] = 0.0
    assert np.max(np.abs(dV_bad.sum(axis=1) - dO_sum)) > 1e-3 * np.max(np.abs(dO_sum))
    assert np.max(np.abs(dK_bad.sum(axis=1)) / np.abs(dK).sum(axis=1)) > 1e-3


def scale_identity_error(dQ, Q, dK, K, G):
    """max over (batch, KV group) of |<dQ, Q> - <dK, K>| / (sum|dQ Q| + sum|dK K|)."""
    B, T, H, D = Q.shape
    Hkv = K.shape[2]
    qq = (dQ * Q).reshape(B, T, Hkv, G, D)
    kk = dK * K
    num = np.abs(qq.sum(axis=(1, 3, 4)) - kk.sum(axis=(1, 3)))
    den = np.abs(qq).sum(axis=(1, 3, 4)) + np.abs(kk).sum(axis=(1, 3))
    return float(np.max(num / np.maximum(den, 1e-300)))


@pytest.mark.parametrize("case", CASES, ids=[str(c[0]) for c in CASES])
def test_backward_scale_identity(case):
    # O(aQ, K/a) = O(Q, K) for every mask, so d/da at a = 1 gives
    # sum <dQ, Q> = sum <dK, K> per (batch, KV group), over every token: the
    # identity the full-size GPU tests check on the whole output.  A planted
    # error (the dQ or the dK of one block of tokens dropped) must break it.
    seed, B, T, H, Hkv, D, window, pos_kind = case
    Q, K, V, dO = rand(seed, B, T, H, Hkv, D)
    pos = _positions(seed, B, T) if pos_kind == "docs" else None
    O, l, m = R.forward(Q, K, V, window, pos)
    dQ, dK, dV = R.backward(dO, Q, K, V, O, l, m, window, pos)
    G = H // Hkv
    assert scale_identity_error(dQ, Q, dK, K, G) < 1e-12
    dQ_bad = dQ.copy()
    dQ_bad[:, T // 2:] = 0.0
    assert scale_identity_error(dQ_bad, Q, dK, K, G) > 1e-4
    dK_bad = dK.copy()
    dK_bad[:, T // 2:] = 0.0
    assert scale_identity_error(dQ, Q, dK_bad, K, G) > 1e-4
    # The fast-mode rounding keeps it to the bf16 rounding of dS.
    gq, gk, _ = R.backward(dO, Q, K, V, O, l, m, window, pos, fast=True)
    assert scale_identity_error(gq, Q, gk, K, G) < 2e-2


def test_round_bf16_matches_torch():
    rng = np.random.Generator(np.random.PCG64(5))
    x = np.concatenate([rng.standard_normal(10000) * 10.0 ** rng.integers(-30, 30, 10000),
                        # exact ties between two bf16 values, both parities
                        np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -(1.0 + 2.0 ** -8), 2.0 ** -130, 0.0, -0.0])])
    x32 = x.astype(np.float32)
    ref = torch.from_numpy(x32).to(torch.bfloat16).to(torch.float64).numpy()
    got = R.round_bf16(x32)
    assert np.array_equal(got.view(np.int64), ref.view(np.int64))


def test_fast_backward_rounding():
    # (a) On inputs whose probabilities and dS are bf16 values the rounding
    # changes nothing: each query sees two keys of equal score (P = 1/2) and
    # dO, V hold small integers (dP - D is then exact in bf16).
    T, D = 8, 16
    Q = np.zeros((1, T, 1, D))
    K = np.zeros((1, T, 1, D))
    rng = np.random.Generator(np.random.PCG64(3))
    V = rng.integers(-3, 4, (1, T, 1, D)).astype(np.float64)
    dO = rng.integers(-3, 4, (1, T, 1, D)).astype(np.float64)
    window = (1, 0)  # keys q-1 and q (query 0 sees one key)
    O, l, m = R.forward(Q, K, V, window)
    exact = R.backward(dO, Q, K, V, O, l, m, window)
    fast = R.backward(dO, Q, K, V, O, l, m, window, fast=True)
    for a, b in zip(fast, exact):
        assert np.array_equal(a, b)
    # (b) In general it moves the gradients by the bf16 rounding of P and dS:
    # about 2^-9 relative, and not zero.
    Q, K, V, dO = rand(4, 1, 40, 2, 1, 32)
    O, l, m = R.forward(Q, K, V, (-1, 0))
    exact = R.backward(dO, Q, K, V, O, l, m, (-1, 0))
    fast = R.backward(dO, Q, K, V, O, l, m, (-1, 0), fast=True)
    for a, b in zip(fast, exact):
        e = max_rel(a, b)
        assert 1e-5 < e < 2e-2
    # (c) dV uses the rounded P and dK the rounded dS: a backward that rounds
    # only dS (P unrounded in dV) differs from it.
    assert max_rel(fast[2], exact[2]) > 1e-5


def test_document_mask_equals_segments():
    T, H, Hkv, D = 30, 2, 1, 16
    lengths = [7, 1, 12, 10]
    pos = np.concatenate([np.arange(n) for n in lengths])[None].astype(np.int32)
    Q, K, V, dO = rand(71, 1, T, H, Hkv, D)
    O, l, m = R.forward(Q, K, V, (-1, 0), pos)
    g = R.backward(dO, Q, K, V, O, l, m, (-1, 0), pos)
    t = 0
    for n in lengths:
        s = slice(t, t + n)
        Os, ls, ms = R.forward(Q[:, s], K[:, s], V[:, s], (-1, 0))
        gs = R.backward(dO[:, s], Q[:, s], K[:, s], V[:, s], Os, ls, ms, (-1, 0))
        assert np.allclose(O[:, s], Os, atol=1e-14)
        for a, b in zip(g, gs):
            assert np.allclose(a[:, s], b, atol=1e-13)
        t += n
    # A row that starts part-way through a document: positions begin above 0.
    pos2 = (pos + 5).astype(np.int32)
    pos2[0, 7:] = pos[0, 7:]
    O2, _, _ = R.forward(Q, K, V, (-1, 0), pos2)
    assert np.allclose(O2[:, :7], O[:, :7], atol=1e-14)


def test_finite_differences_toy_config():
    """Central differences of L = sum(dO . O) on the README toy shapes (C1)."""
    wl = W.WORKLOADS["C1"]
    h = W.host_inputs(wl)
    Q, K, V, dO = (x.astype(np.float64) for x in (h.Q, h.K, h.V, h.dO))
    O, l, m = R.forward(Q, K, V, h.window)
    grads = R.backward(dO, Q, K, V, O, l, m, h.window)
    eps = 1e-6
    for idx, X in enumerate((Q, K, V)):
        num = np.zeros_like(X)
        it = np.nditer(X, flags=["multi_index"])
        for _ in it:
            i = it.multi_index
            Xp, Xm = X.copy(), X.copy()
            Xp[i] += eps
            Xm[i] -= eps
            args_p = [Q, K, V]
            args_m = [Q, K, V]
            args_p[idx], args_m[idx] = Xp, Xm
            Lp = np.sum(dO * R.forward(*args_p, h.window)[0])
            Lm = np.sum(dO * R.forward(*args_m, h.window)[0])
            num[i] = (Lp - Lm) / (2 * eps)
        assert max_rel(grads[idx], num) < 1e-6


@pytest.mark.parametrize("window,T,pos", [((-1, 0), 700, False), ((100, 0), 600, False), ((50, 20), 530, False),
                                          ((-1, 0), 650, True)])
def test_fa1_restatement_matches_oracle(window, T, pos):
    B, H, Hkv, D = 2, 4, 2, 32
    Q, K, V, dO = (x.astype(np.float32) for x in rand(81 + T, B, T, H, Hkv, D))
    positions = W.document_positions(T, B, seed=T, mean=150, sigma=1.0, cap=400) if pos else None
    O, l, m = R.forward(Q, K, V, window, positions)
    O1, l1, m1 = fa1.forward(Q, K, V, window, positions, nthreads=4)
    assert max_rel(O1, O) < 1e-5
    assert np.max(np.abs(R.lse(l1, m1) - R.lse(l, m))) < 1e-5
    g = R.backward(dO, Q, K, V, O, l, m, window, positions)
    g1 = fa1.backward(dO, Q, K, V, O1, l1, m1, window, positions, nthreads=4)
    for a, b in zip(g1, g):
        assert max_rel(a, b) < 1e-5
    # The restatement accumulates like Δflash_attention₁!.
    g2 = fa1.backward(dO, Q, K, V, O1, l1, m1, window, positions, nthreads=4, dQ=g1[0].copy(), dK=g1[1].copy(),
                      dV=g1[2].copy())
    for a, b in zip(g2, g1):
        assert max_rel(a, 2 * b) < 1e-5  # fp32 sums in a different order


@pytest.mark.parametrize("window,T,pos", [((-1, 0), 700, False), ((100, 0), 600, False), ((50, 20), 530, False),
                                          ((-1, 0), 650, True)])
def test_blas_restatement_matches_oracle(window, T, pos):
    # oracle/fa1_blas.py, the CPU baseline bench.py times: the reference's
    # blocked algorithm with BLAS products, float32.
    B, H, Hkv, D = 2, 4, 2, 32
    Q, K, V, dO = (x.astype(np.float32) for x in rand(91 + T, B, T, H, Hkv, D))
    positions = W.document_positions(T, B, seed=T, mean=150, sigma=1.0, cap=400) if pos else None
    O, l, m = R.forward(Q, K, V, window, positions)
    O1, l1, m1 = fa1_blas.forward(Q, K, V, window, positions)
    assert max_rel(O1, O) < 1e-5
    assert np.max(np.abs(R.lse(l1, m1) - R.lse(l, m))) < 1e-5
    g = R.backward(dO, Q, K, V, O, l, m, window, positions)
    g1 = fa1_blas.backward(dO, Q, K, V, O1, l1, m1, window, positions)
    for a, b in zip(g1, g):
        assert max_rel(a, b) < 1e-5
    # It accumulates like Δflash_attention₁!.
    g2 = fa1_blas.backward(dO, Q, K, V, O1, l1, m1, window, positions, *(x.copy() for x in g1))
    for a, b in zip(g2, g1):
        assert max_rel(a, 2 * b) < 1e-5
    # Its statistics are the reference's: m the row max over visible keys.
    assert max_rel(m1[l > 0], m[l > 0]) < 1e-6


def test_golden_fixture_c1():
    """The committed C1 vectors (generated by tests/golden/make_golden.py) are reproduced."""
    z = np.load(GOLDEN)
    wl = W.WORKLOADS["C1"]
    h = W.host_inputs(wl)
    assert np.array_equal(h.Q, z["Q"]) and np.array_equal(h.K, z["K"]) and np.array_equal(h.V, z["V"])
    O, l, m = R.forward(z["Q"], z["K"], z["V"], tuple(z["window"]), z["positions"])
    assert np.allclose(O, z["O"], rtol=0, atol=1e-12)
    assert np.allclose(l, z["l"], rtol=0, atol=1e-12) and np.allclose(m, z["m"], rtol=0, atol=1e-12)
    g = R.backward(z["dO"], z["Q"], z["K"], z["V"], z["O"], z["l"], z["m"], tuple(z["window"]), z["positions"])
    for name, x in zip(("dQ", "dK", "dV"), g):
        assert np.allclose(x, z[name], rtol=0, atol=1e-12)


def test_golden_fixture_slice():
    """The committed C3-shaped slice (document mask, window (20,0), bf16 inputs) is reproduced."""
    z = np.load(SLICE_GOLDEN)
    window = tuple(int(w) for w in z["window"])
    O, l, m = R.forward(z["Q"], z["K"], z["V"], window, z["positions"])
    assert np.allclose(O, z["O"], rtol=0, atol=1e-6)  # stored as float32
    assert np.allclose(l, z["l"], rtol=0, atol=1e-12) and np.allclose(m, z["m"], rtol=0, atol=1e-12)
    g = R.backward(z["dO"], z["Q"], z["K"], z["V"], O, l, m, window, z["positions"])
    for name, x in zip(("dQ", "dK", "dV"), g):
        assert np.allclose(x, z[name], rtol=0, atol=1e-6 * max(1.0, float(np.abs(x).max())))
    # bf16 inputs: every value is a bfloat16 number
    for name in ("Q", "K", "V", "dO"):
        assert np.array_equal(R.round_bf16(z[name]), z[name].astype(np.float64))


PLANTED = {
    "no_scale": lambda Q, K, V, w, p: R.forward(Q * np.sqrt(Q.shape[-1]), K, V, w, p),
    "transposed_keys": lambda Q, K, V, w, p: R.forward(Q, K[:, ::-1].copy(), V, w, p),
    "window_off_by_one": lambda Q, K, V, w, p: R.forward(Q, K, V, (w[0] - 1, w[1]), p),
    "wrong_gqa_map": lambda Q, K, V, w, p: R.forward(Q[:, :, ::-1].copy(), K, V, w, p),
}


@pytest.mark.parametrize("name", sorted(PLANTED))
def test_planted_mistakes_are_caught(name):
    """A plausible mistake planted in the oracle fails the independent check."""
    B, T, H, Hkv, D = 1, 12, 4, 2, 16
    Q, K, V, dO = rand(91, B, T, H, Hkv, D)
    window = (5, 0)
    O_bad = PLANTED[name](Q, K, V, window, None)[0]
    O_t = torch_reference(Q, K, V, dO, window)[0]
    assert max_rel(O_bad, O_t) > 1e-3
