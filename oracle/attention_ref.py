"""Dense float64 restatement of femtochat's attention (the parity oracle).

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import this package, and only as the checker;
the product path (femtochat_amd) never calls it.

What is restated (all file:line citations are into msjgriffiths/femtochat):

* ``visible``      : the mask of ``attention_mask!`` (src/kernels.jl:30-42):
  causal ``k <= q`` when window == (-1, 0), otherwise ``q-left <= k <= q+right``;
  plus the document rule ``k >= q - positions[q]`` when positions are given
  (a new feature; positions restart at 0 per document, src/dataloader.jl:157-174).
* ``forward``      : ``naive_attention`` (src/kernels.jl:59-96) with the
  statistics of ``flash_attention₁!`` (src/kernels.jl:131-219):
  m = max of the visible scaled scores (natural log), l = sum exp(S - m); a
  query with no visible key keeps m = -floatmax, l = 0, O = 0.
* ``backward``     : ``Δflash_attention₁!`` (src/kernels.jl:287-379):
  P = exp(S - m) / max(l, eps(Float32)), dV += dO P^T, dP = dO V^T,
  D = rowsum(dO . O), dS = P (dP - D), dQ += tau K dS, dK += tau Q dS^T.

Arrays use the torch layout of the library: Q, O, dO (B, T, H, D); K, V
(B, T, Hkv, D); l, m (B, H, T); positions (B, T).  GQA maps 0-based head h to
KV head h // (H // Hkv) (src/kernels.jl:69,161,318: ``cld(head, H÷Hkv)``).

Pinning (tests/test_oracle.py): torch.autograd through an independent
softmax/matmul formulation and torch's scaled_dot_product_attention, central
finite differences on the toy config, the C float32 FA-1 restatement
(oracle/fa1.c), and the closed forms and invariants listed there.
"""
from __future__ import annotations

import numpy as np

FLT_MAX = float(np.finfo(np.float32).max)
EPS_F32 = float(np.finfo(np.float32).eps)


def visible(T: int, window, positions_row=None) -> np.ndarray:
    """Bool [q, k]: key k visible to query q (0-based token indices)."""
    q = np.arange(T)[:, None]
    k = np.arange(T)[None, :]
    left, right = int(window[0]), int(window[1])
    if (left, right) == (-1, 0):
        vis = k <= q
    else:
        vis = (q - left <= k) & (k <= q + right)
    if positions_row is not None:
        pos = np.asarray(positions_row, dtype=np.int64)
        vis = vis & (k >= (q - pos[:, None]))
    return vis


def _f64(x):
    return np.asarray(x, dtype=np.float64)


def forward(Q, K, V, window, positions=None):
    """Returns (O, l, m) in float64."""
    Q, K, V = _f64(Q), _f64(K), _f64(V)
    B, T, H, D = Q.shape
    Hkv = K.shape[2]
    G = H // Hkv
    tau = 1.0 / np.sqrt(D)
    O = np.zeros((B, T, H, D))
    l = np.zeros((B, H, T))
    m = np.full((B, H, T), -FLT_MAX)
    for b in range(B):
        vis = visible(T, window, None if positions is None else positions[b])
        has = vis.any(axis=1)
        for h in range(H):
            kv = h // G
            S = (Q[b, :, h, :] @ K[b, :, kv, :].T) * tau
            Sm = np.where(vis, S, -np.inf)
            mrow = np.where(has, Sm.max(axis=1, initial=-np.inf), 0.0)
            P = np.where(vis, np.exp(np.where(vis, S, 0.0) - mrow[:, None]), 0.0)
            lrow = P.sum(axis=1)
            O[b, :, h, :] = (P / np.where(lrow > 0, lrow, 1.0)[:, None]) @ V[b, :, kv, :]
            l[b, h] = lrow
            m[b, h] = np.where(has, mrow, -FLT_MAX)
    return O, l, m


def round_bf16(x) -> np.ndarray:
    """x rounded to bfloat16 (through float32, then to nearest even), as
    float64 values: the rounding the fast kernels apply to fp32 values."""
    f = np.asarray(x, dtype=np.float64).astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).astype(np.float64)


def backward(dO, Q, K, V, O, l, m, window, positions=None, fast=False):
    """Returns (dQ, dK, dV) in float64 (the increments Δflash_attention₁! adds).

    fast=True restates the rounding of the reference's tensor-core backward
    (ext/FemtoChatCUDAExt.jl:1915-1946): P is rounded to bf16 before
    dV += P^T dO, dS = P (dP - D) is formed from the unrounded P and rounded to
    bf16 before both dK and dQ, and a query with a single visible key has
    dS = 0 (:1929-1930)."""
    dO, Q, K, V, O, l, m = map(_f64, (dO, Q, K, V, O, l, m))
    B, T, H, D = Q.shape
    Hkv = K.shape[2]
    G = H // Hkv
    tau = 1.0 / np.sqrt(D)
    dQ = np.zeros_like(Q)
    dK = np.zeros_like(K)
    dV = np.zeros_like(V)
    for b in range(B):
        vis = visible(T, window, None if positions is None else positions[b])
        for h in range(H):
            kv = h // G
            S = (Q[b, :, h, :] @ K[b, :, kv, :].T) * tau
            with np.errstate(over="ignore"):  # rows with no visible key: m = -floatmax, P = 0
                P = np.where(vis, np.exp(np.where(vis, S, 0.0) - m[b, h][:, None]), 0.0)
            P = P / np.maximum(l[b, h], EPS_F32)[:, None]
            dOh = dO[b, :, h, :]
            dV[b, :, kv, :] += (round_bf16(P) if fast else P).T @ dOh
            dP = dOh @ V[b, :, kv, :].T
            Dq = (dOh * O[b, :, h, :]).sum(axis=1)
            dS = P * (dP - Dq[:, None])
            if fast:
                dS = round_bf16(np.where((vis.sum(axis=1) > 1)[:, None], dS, 0.0))
            dQ[b, :, h, :] += tau * (dS @ K[b, :, kv, :])
            dK[b, :, kv, :] += tau * (dS.T @ Q[b, :, h, :])
    return dQ, dK, dV


def lse(l, m):
    """Natural-log log-sum-exp L = m + log(l) (row statistics of the forward)."""
    l, m = _f64(l), _f64(m)
    with np.errstate(divide="ignore"):
        return m + np.log(l)


def visible_pairs(T: int, B: int, H: int, window, positions=None) -> int:
    """Number of visible (query, key) pairs over all rows and heads."""
    total = 0
    for b in range(B):
        total += int(visible(T, window, None if positions is None else positions[b]).sum())
    return total * H
