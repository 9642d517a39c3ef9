"""Shared helpers for the parity tests (comparison metrics, GPU runners)."""
from __future__ import annotations

import sys

import numpy as np

# Tolerances of the parity contract: max|X-R| / max|R| per output tensor,
# and the natural-log log-sum-exp L = m + log(l) in absolute terms.
TOL = {"exact": 1e-4, "fast": 2e-2}
TOL_LSE = 1e-5


# Outputs that are mathematically zero (dQ when every query sees only
# itself) leave only rounding noise in the reference; the denominator of the
# relative error is floored at this absolute value.
ABS_FLOOR = 1e-6


def rel_err(x, ref, floor: float = ABS_FLOOR) -> float:
    """max|x - ref| / max(max|ref|, floor)."""
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    if ref.size == 0:
        return 0.0
    scale = max(float(np.max(np.abs(ref))), floor)
    return float(np.max(np.abs(x - ref))) / scale


def lse_err(l, m, l_ref, m_ref) -> float:
    """max |L - L_ref| over queries with at least one visible key."""
    l, m, l_ref, m_ref = (np.asarray(a, np.float64) for a in (l, m, l_ref, m_ref))
    has = l_ref > 0
    if not has.any():
        return 0.0
    L = m[has] + np.log(l[has])
    R = m_ref[has] + np.log(l_ref[has])
    return float(np.max(np.abs(L - R)))


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


def to_np(t):
    import torch

    return t.detach().to(torch.float32).cpu().numpy()


def gpu_forward(A, Q, K, V, window, positions=None, out_dtype=None):
    import torch

    from femtochat_amd import kernels as Kn

    B, T, H, D = Q.shape
    O = torch.empty(Q.shape, dtype=out_dtype or Q.dtype, device=Q.device)
    l = torch.empty((B, H, T), dtype=torch.float32, device=Q.device)
    m = torch.empty((B, H, T), dtype=torch.float32, device=Q.device)
    Kn.attention_(A, O, l, m, Q, K, V, window, positions=positions)
    return O, l, m


def gpu_backward(A, dO, Q, K, V, O, l, m, window, positions=None, grad_dtype=None, accumulate=False, init=None):
    import torch

    from femtochat_amd import kernels as Kn

    gd = grad_dtype or Q.dtype
    if init is None:
        dQ = torch.zeros(Q.shape, dtype=gd, device=Q.device)
        dK = torch.zeros(K.shape, dtype=gd, device=Q.device)
        dV = torch.zeros(V.shape, dtype=gd, device=Q.device)
    else:
        dQ, dK, dV = (x.clone() for x in init)
    Kn.delta_attention_(A, dQ, dK, dV, dO, Q, K, V, O, l, m, window, positions=positions, accumulate=accumulate)
    return dQ, dK, dV
