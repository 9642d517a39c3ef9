"""The reference's blocked CPU attention with BLAS products (numpy float32).

TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times it on the host
cores and tests/test_oracle.py checks it against the float64 oracle; nothing
in femtochat_amd calls it.

It restates ``flash_attention₁!`` (src/kernels.jl:131-219) and
``Δflash_attention₁!`` (src/kernels.jl:287-379) step by step, with the same
loop nest (document and head outer, 512-wide key blocks j, then 512-wide query
blocks i), no block skipping, every product a BLAS sgemm as the reference's
``mul!`` calls are (there: OpenBLAS through LinearAlgebra; here: numpy's
BLAS), and the element-wise steps as whole-block array operations (the
reference's broadcasts):

  forward, per block pair:  S = K_j^T Q_i * scale (:190-191), masked to
  -floatmax (:193-194), m~ = column max (:196), P~ = mask ? exp(S - m~) : 0
  (:197), l~ = column sum (:199), the running (m, l) update (:201-204),
  O~ = V_j P~ (:206) and O = (O l e^(m-m_new) + O~ e^(m~-m_new)) / max(l_new, eps)
  (:207-210).
  backward, per block pair: P = mask ? exp(S - m) / max(l, eps) : 0 (:346-354),
  dV_j += dO_i P^T (:358), dP = V_j^T dO_i (:361), D = rowsum(dO_i . O_i)
  (:364-365), dS = P (dP - D) (:368), dQ_i += scale K_j dS (:371),
  dK_j += scale Q_i dS^T (:374).

Arrays use the library's torch layout (row-major): Q, O, dO (B, T, H, D);
K, V (B, T, Hkv, D); l, m (B, H, T).  ``positions`` (B, T) adds the document
rule k >= q - positions[q], which the reference does not have (its
``attention_mask!``, src/kernels.jl:30-42, is the window rule only).
"""
from __future__ import annotations

import numpy as np

BLOCK = 512
_F = np.float32
_MASKED = np.float32(-np.finfo(np.float32).max)
_EPS = np.float32(np.finfo(np.float32).eps)


def _mask(j0, nj, i0, ni, window, pos_row):
    """attention_mask!(M, keys, queries, window): M[key, query] (src/kernels.jl:30-42)."""
    key = np.arange(j0, j0 + nj)[:, None]
    query = np.arange(i0, i0 + ni)[None, :]
    left, right = int(window[0]), int(window[1])
    if (left, right) == (-1, 0):
        M = key <= query
    else:
        M = (query - left <= key) & (key <= query + right)
    if pos_row is not None:
        M = M & (key >= query - pos_row[i0:i0 + ni][None, :].astype(np.int64))
    return M


def forward(Q, K, V, window, positions=None):
    """Returns (O, l, m) in float32, the outputs of flash_attention₁!."""
    Q, K, V = (np.ascontiguousarray(x, dtype=_F) for x in (Q, K, V))
    B, T, H, D = Q.shape
    G = H // K.shape[2]
    scale = _F(1.0 / np.sqrt(_F(D)))
    O = np.zeros((B, T, H, D), _F)
    l = np.zeros((B, H, T), _F)
    m = np.full((B, H, T), -np.inf, _F)  # typemin(F)
    for b in range(B):
        pos_row = None if positions is None else positions[b]
        for h in range(H):
            kv = h // G
            for j0 in range(0, T, BLOCK):
                nj = min(BLOCK, T - j0)
                Kj = K[b, j0:j0 + nj, kv]
                Vj = V[b, j0:j0 + nj, kv]
                for i0 in range(0, T, BLOCK):
                    ni = min(BLOCK, T - i0)
                    Qi = Q[b, i0:i0 + ni, h]
                    mi, li = m[b, h, i0:i0 + ni], l[b, h, i0:i0 + ni]
                    S = Kj @ Qi.T
                    S *= scale
                    M = _mask(j0, nj, i0, ni, window, pos_row)
                    S = np.where(M, S, _MASKED)
                    mt = S.max(axis=0)
                    with np.errstate(over="ignore"):  # masked entries: -floatmax - m~
                        P = np.where(M, np.exp(S - mt), _F(0))
                    lt = P.sum(axis=0, dtype=_F)
                    mn = np.maximum(mi, mt)
                    em, emt = np.exp(mi - mn), np.exp(mt - mn)
                    ln = em * li + emt * lt
                    Ot = Vj.T @ P  # (D, ni)
                    O[b, i0:i0 + ni, h] = (O[b, i0:i0 + ni, h] * (li * em)[:, None] + Ot.T * emt[:, None]) / \
                        np.maximum(ln, _EPS)[:, None]
                    m[b, h, i0:i0 + ni] = mn
                    l[b, h, i0:i0 + ni] = ln
    return O, l, m


def backward(dO, Q, K, V, O, l, m, window, positions=None, dQ=None, dK=None, dV=None):
    """Adds the gradients into dQ, dK, dV (zeros when not given) as
    Δflash_attention₁! does, and returns them (float32)."""
    dO, Q, K, V, O, l, m = (np.ascontiguousarray(x, dtype=_F) for x in (dO, Q, K, V, O, l, m))
    B, T, H, D = Q.shape
    G = H // K.shape[2]
    scale = _F(1.0 / np.sqrt(_F(D)))
    dQ = np.zeros_like(Q) if dQ is None else dQ
    dK = np.zeros_like(K) if dK is None else dK
    dV = np.zeros_like(V) if dV is None else dV
    for b in range(B):
        pos_row = None if positions is None else positions[b]
        for h in range(H):
            kv = h // G
            for j0 in range(0, T, BLOCK):
                nj = min(BLOCK, T - j0)
                Kj, Vj = K[b, j0:j0 + nj, kv], V[b, j0:j0 + nj, kv]
                for i0 in range(0, T, BLOCK):
                    ni = min(BLOCK, T - i0)
                    Qi, Oi, dOi = Q[b, i0:i0 + ni, h], O[b, i0:i0 + ni, h], dO[b, i0:i0 + ni, h]
                    mi, li = m[b, h, i0:i0 + ni], l[b, h, i0:i0 + ni]
                    S = Kj @ Qi.T
                    S *= scale
                    M = _mask(j0, nj, i0, ni, window, pos_row)
                    S = np.where(M, S, _MASKED)
                    with np.errstate(over="ignore"):
                        P = np.where(M, np.exp(S - mi) / np.maximum(li, _EPS), _F(0))
                    dV[b, j0:j0 + nj, kv] += P @ dOi
                    dP = Vj @ dOi.T
                    Dr = (dOi * Oi).sum(axis=1, dtype=_F)
                    dS = P * (dP - Dr)
                    dQ[b, i0:i0 + ni, h] += scale * (dS.T @ Kj)
                    dK[b, j0:j0 + nj, kv] += scale * (dS @ Qi)
    return dQ, dK, dV


def blas_info() -> dict:
    """The BLAS numpy uses and its thread count (threadpoolctl)."""
    try:
        from threadpoolctl import threadpool_info
    except ImportError:  # pragma: no cover
        return {}
    for p in threadpool_info():
        if p.get("user_api") == "blas":
            return {"library": p.get("internal_api"), "version": p.get("version"), "threads": p.get("num_threads")}
    return {}
