"""ctypes wrapper of oracle/fa1.c (float32 FA-1 restatement) — test infrastructure."""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_LIB = None
_PATH = Path(__file__).resolve().parent / "liboracle_fa1.so"


def _lib():
    global _LIB
    if _LIB is None:
        if not _PATH.exists():
            from . import build

            build.build()
        lib = ctypes.CDLL(str(_PATH))
        P = ctypes.c_void_p
        i = ctypes.c_int
        lib.fa1_forward.argtypes = [P, P, P, P, P, P, P] + [i] * 9
        lib.fa1_forward.restype = None
        lib.fa1_backward.argtypes = [P] * 11 + [i] * 9
        lib.fa1_backward.restype = None
        _LIB = lib
    return _LIB


def _c(x, dtype):
    a = np.ascontiguousarray(x, dtype=dtype)
    return a, a.ctypes.data_as(ctypes.c_void_p)


def _window_args(window):
    left, right = int(window[0]), int(window[1])
    causal = int((left, right) == (-1, 0))
    return left, right, causal


def forward(Q, K, V, window, positions=None, nthreads=0):
    """float32 (O, l, m) of the blocked FA-1 forward (src/kernels.jl:131-219)."""
    Q, qp = _c(Q, np.float32)
    K, kp = _c(K, np.float32)
    V, vp = _c(V, np.float32)
    B, T, H, D = Q.shape
    Hkv = K.shape[2]
    pos, pp = (None, None) if positions is None else _c(positions, np.int32)
    O = np.zeros((B, T, H, D), np.float32)
    l = np.zeros((B, H, T), np.float32)
    m = np.zeros((B, H, T), np.float32)
    left, right, causal = _window_args(window)
    _lib().fa1_forward(qp, kp, vp, pp, O.ctypes.data_as(ctypes.c_void_p), l.ctypes.data_as(ctypes.c_void_p),
                       m.ctypes.data_as(ctypes.c_void_p), D, H, Hkv, T, B, left, right, causal, int(nthreads))
    return O, l, m


def backward(dO, Q, K, V, O, l, m, window, positions=None, nthreads=0, dQ=None, dK=None, dV=None):
    """float32 (dQ, dK, dV) of the blocked FA-1 backward (src/kernels.jl:287-379).
    Accumulates into dQ/dK/dV when given (zeros otherwise)."""
    arrs = [_c(x, np.float32) for x in (dO, Q, K, V, O, l, m)]
    Qa = arrs[1][0]
    B, T, H, D = Qa.shape
    Hkv = arrs[2][0].shape[2]
    pos, pp = (None, None) if positions is None else _c(positions, np.int32)
    dQ = np.zeros((B, T, H, D), np.float32) if dQ is None else np.ascontiguousarray(dQ, np.float32)
    dK = np.zeros((B, T, Hkv, D), np.float32) if dK is None else np.ascontiguousarray(dK, np.float32)
    dV = np.zeros((B, T, Hkv, D), np.float32) if dV is None else np.ascontiguousarray(dV, np.float32)
    left, right, causal = _window_args(window)
    _lib().fa1_backward(*[p for _, p in arrs], pp, dQ.ctypes.data_as(ctypes.c_void_p),
                        dK.ctypes.data_as(ctypes.c_void_p), dV.ctypes.data_as(ctypes.c_void_p),
                        D, H, Hkv, T, B, left, right, causal, int(nthreads))
    return dQ, dK, dV
