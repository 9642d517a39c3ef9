"""Restatement of femtochat's optimizer kernels (the parity oracle for them).

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import this package, and only as the checker;
the product path (femtochat_amd) never calls it.

What is restated (citations into msjgriffiths/femtochat):

* ``julia_pow_f32``  : Julia's ``Float32 ^ Int`` as the AdamW bias corrections
  use it (``β₁^t``): ``x*x*x`` in Float32 for t = 3, otherwise
  square-and-multiply in Float64 rounded to Float32.
* ``adamw_step``     : ``adam_moments!`` (src/optim.jl:32-38) then the update
  of ``(ω::AdamW)(θ, g)`` (:82-94), operation by operation in float32 (Julia
  does not fuse multiply-adds).
* ``adam_update``    : the CUDA final write ``adam_update_kernel!``
  (ext/FemtoChatCUDAExt.jl:99-106): θ = θ (1 - η λ) - α m / (sqrt(v / β) + ϵ).
* ``muon_update``    : ``muon_update_kernel!`` (CUDAExt:108-119) and the generic
  ``(ω::Muon)`` write (src/optim.jl:238-247): θ -= η x + η λ θ [x θ >= 0]
  (cautious weight decay), on the flat storage at per-matrix offsets.
* ``gather`` / ``scatter`` : ``gather!`` / ``scatter!`` (src/optim.jl:262-276,
  CUDAExt:127-149).
* ``polar_express``  : ``polar_express!`` (src/optim.jl:115-149) in float64.

Arrays are numpy; matrices use the reference's column-major convention via
numpy's order="F" views where it matters (polar_express takes (k, m, n)
stacks whose [k] is the Julia matrix G[:, :, k]).

Pinning (tests/test_optim_oracle.py): torch.optim.AdamW's formula in
float64, the t = 1 closed form, Julia's power against float64 pow, the two
branches of the cautious decay, and for Polar Express the singular value
decomposition (the iteration applies the composed polynomial to the singular
values), transposition, and planted mistakes.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32

# (a, b, c) per Polar Express step (src/optim.jl:97-103), as float32 values.
COEFFICIENTS = (
    (8.156554524902461, -22.48329292557795, 15.878769915207462),
    (4.042929935166739, -2.808917465908714, 0.5000178451051316),
    (3.8916678022926607, -2.772484153217685, 0.5060648178503393),
    (3.285753657755655, -2.3681294933425376, 0.46449024233003106),
    (2.3465413258596377, -1.7097828382687081, 0.42323551169305323),
)


def julia_pow_f32(x, t: int) -> np.float32:
    """Julia's ``x::Float32 ^ t::Int`` for t >= 1."""
    x = F32(x)
    if t == 3:
        return F32(F32(x * x) * x)
    # square-and-multiply in Float64 (Base.power_by_squaring)
    y, b, p = 1.0, float(x), int(t)
    first = True
    while p > 0:
        if p & 1:
            y = b if first else y * b
            first = False
        p >>= 1
        if p:
            b = b * b
    return F32(y)


def adamw_step(theta, g, m, v, t, alpha, beta1, beta2, eps, lam, grad_scale=1.0):
    """One AdamW step at step count t (after the increment); returns new
    (theta, m, v) as float32 arrays, every operation rounded to float32."""
    th, g, m, v = (np.asarray(a, F32) for a in (theta, g, m, v))
    a, b1, b2, e, l, n = (F32(x) for x in (alpha, beta1, beta2, eps, lam, grad_scale))
    gn = g / n
    m = b1 * m + (F32(1) - b1) * gn
    v = b2 * v + (F32(1) - b2) * (gn * gn)
    th = th * (F32(1) - a * l)
    c1 = F32(1) - julia_pow_f32(b1, t)
    c2 = F32(1) - julia_pow_f32(b2, t)
    th = th - (a * (m / c1)) / (np.sqrt(v / c2) + e)
    return th.astype(F32), m.astype(F32), v.astype(F32)


def adam_update(Theta, offset, m, v, alpha, beta, eta, lam, eps):
    """The CUDA final write into the flat Theta (a new array)."""
    Th = np.array(Theta, F32, copy=True)
    m, v = np.asarray(m, F32), np.asarray(v, F32)
    a, b, h, l, e = (F32(x) for x in (alpha, beta, eta, lam, eps))
    sl = slice(offset, offset + m.size)
    Th[sl] = Th[sl] * (F32(1) - h * l) - (a * m) / (np.sqrt(v / b) + e)
    return Th


def muon_update(Theta, X, offsets, eta, lam):
    """Cautious update of each stacked matrix into the flat Theta: X is
    (k, width) (matrix j's elements in the reference's order)."""
    Th = np.array(Theta, F32, copy=True)
    X = np.asarray(X, F32)
    h, l = F32(eta), F32(lam)
    for j, off in enumerate(offsets):
        sl = slice(int(off), int(off) + X.shape[1])
        th, x = Th[sl], X[j]
        decay = (h * l) * th
        decay = np.where(x * th >= 0, decay, np.copysign(F32(0), decay))
        Th[sl] = th - (h * x + decay)
    return Th


def gather(vector, offsets, width):
    v = np.asarray(vector)
    return np.stack([v[int(o):int(o) + width] for o in offsets])


def scatter(vector, stack, offsets):
    out = np.array(vector, copy=True)
    for j, o in enumerate(offsets):
        out[int(o):int(o) + stack.shape[1]] = stack[j]
    return out


def polar_express(G, steps: int = 5, coefficients=COEFFICIENTS):
    """polar_express! on a (k, m, n) stack of matrices, float64."""
    G = np.asarray(G, np.float64)
    out = np.empty_like(G)
    for j in range(G.shape[0]):
        g = G[j]
        transposed = g.shape[0] > g.shape[1]
        scale = float(F32(1.01)) * np.sqrt(np.sum(g * g)) + float(F32(1e-6))
        X = (g.T if transposed else g) / scale
        for t in range(steps):
            a, b, c = (float(F32(x)) for x in coefficients[min(t, len(coefficients) - 1)])
            A = X @ X.T
            B = b * A + c * (A @ A)
            X = a * X + B @ X
        out[j] = X.T if transposed else X
    return out


def composed_polynomial(s, steps: int = 5, coefficients=COEFFICIENTS):
    """The scalar map that polar_express applies to each normalised singular value."""
    s = np.asarray(s, np.float64)
    for t in range(steps):
        a, b, c = (float(F32(x)) for x in coefficients[min(t, len(coefficients) - 1)])
        s = a * s + b * s ** 3 + c * s ** 5
    return s
