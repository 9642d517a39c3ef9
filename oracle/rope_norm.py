"""Restatement of femtochat's attention prologue (the parity oracle for it).

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import this package, and only as the checker;
the product path (femtochat_amd) never calls it.

What is restated (citations into msjgriffiths/femtochat):

* ``tables``   : ``rotary_embeddings`` (src/parameters.jl:409-427): for
  channel j < D/2 and position t, angle t * inv_freq[j] with
  inv_freq[j] = 1 / base^(2j / D) (base 1e5); sin and cos tables, Float32.
* ``forward``  : ``apply_rotary_embedding`` (src/gpt.jl:53-77) then
  ``norm`` (src/gpt.jl:15-20) scaled by 1.2 (src/gpt.jl:103-106), with the
  table column of the token's position (``rotary_factors``, src/gpt.jl:43-49):
      u[j]   =  x[j] c[j] + x[j+d] s[j],   u[j+d] = -x[j] s[j] + x[j+d] c[j]
      y      =  u / sqrt(sum(u^2)/D + eps) * 1.2,   eps = eps(eltype(x)).
  Three arithmetic modes: ``"f64"`` (the mathematics), ``"f32"`` (every
  operation in float32, no fused multiply-add, as Julia evaluates Float32),
  ``"bf16"`` (Julia's BFloat16: the tables converted to bf16 (gpt.jl:64-66),
  every product and sum of the rotation rounded to bf16, the norm's sum of
  squares and division in float32 then rounded (gpt.jl:18), the product by
  1.2f0 in float32 then rounded (gpt.jl:105)).
* ``backward`` : the gradient of the f64 function (J^T dY) for given tables.

Arrays use the library's torch layout: X (B, T, NH, D), tables (L, D/2),
positions (B, T).

Pinning (tests/test_prologue_oracle.py): the rotation against complex
multiplication by exp(-i angle); position 0 against the plain norm; the
closed form of the output RMS; central finite differences for the backward;
bf16 rounding against torch's float32 -> bfloat16 conversion, and the f32
mode against torch's float32 elementwise arithmetic; planted mistakes must
fail one of these.
"""
from __future__ import annotations

import numpy as np

EPS = {"f64": float(np.finfo(np.float32).eps), "f32": np.float32(np.finfo(np.float32).eps),
       "bf16": np.float32(2.0 ** -7)}


def bf16_round(x) -> np.ndarray:
    """float32 -> bfloat16 (round to nearest, ties to even) -> float32."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def tables(seq_len: int, head_dim: int, base: float = 100_000.0):
    """(sin, cos), each (seq_len, head_dim // 2) float32."""
    j = np.arange(0, head_dim, 2, dtype=np.float64)
    inv_freq = (1.0 / base ** (j / head_dim)).astype(np.float32)
    t = np.arange(seq_len, dtype=np.float32)
    freqs = t[:, None] * inv_freq[None, :]  # float32 products
    return np.sin(freqs.astype(np.float64)).astype(np.float32), np.cos(freqs.astype(np.float64)).astype(np.float32)


def _columns(sin, cos, B, T, positions):
    """Per-token table columns (B, T, 1, d); NaN for positions out of range."""
    pos = np.broadcast_to(np.arange(T)[None, :], (B, T)) if positions is None else np.asarray(positions)
    L = sin.shape[0]
    ok = (pos >= 0) & (pos < L)
    idx = np.where(ok, pos, 0)
    s = np.where(ok[..., None], sin[idx], np.nan)[:, :, None, :]
    c = np.where(ok[..., None], cos[idx], np.nan)[:, :, None, :]
    return s, c


def rotate(X, sin, cos, positions=None, mode: str = "f64"):
    """u = apply_rotary_embedding(X) (src/gpt.jl:53-77) in the given arithmetic."""
    B, T, NH, D = X.shape
    d = D // 2
    s, c = _columns(sin, cos, B, T, positions)
    if mode == "f64":
        x = np.asarray(X, dtype=np.float64)
        s, c = s.astype(np.float64), c.astype(np.float64)
        x1, x2 = x[..., :d], x[..., d:]
        return np.concatenate([x1 * c + x2 * s, x1 * -s + x2 * c], axis=-1)
    x = np.asarray(X, dtype=np.float32)
    x1, x2 = x[..., :d], x[..., d:]
    s, c = s.astype(np.float32), c.astype(np.float32)
    if mode == "f32":
        return np.concatenate([(x1 * c) + (x2 * s), (x1 * -s) + (x2 * c)], axis=-1).astype(np.float32)
    if mode == "bf16":
        s, c = bf16_round(s), bf16_round(c)
        r = bf16_round
        return np.concatenate([r(r(x1 * c) + r(x2 * s)), r(r(x1 * -s) + r(x2 * c))], axis=-1)
    raise ValueError(mode)


def forward(X, sin, cos, positions=None, mode: str = "f64") -> np.ndarray:
    """Y = norm(apply_rotary_embedding(X)) .* 1.2 (src/gpt.jl:15-20, 103-106)."""
    D = X.shape[-1]
    u = rotate(X, sin, cos, positions, mode)
    eps = EPS[mode]
    if mode == "f64":
        r = np.sqrt(np.sum(u * u, axis=-1, keepdims=True) / D + eps)
        return u / r * 1.2
    ss = np.sum(u * u, axis=-1, keepdims=True, dtype=np.float32)
    r = np.sqrt(ss / np.float32(D) + eps).astype(np.float32)
    if mode == "f32":
        return ((u / r) * np.float32(1.2)).astype(np.float32)
    return bf16_round(bf16_round(u / r) * np.float32(1.2))


def backward(dY, X, sin, cos, positions=None, rotation_mode: str = "f64") -> np.ndarray:
    """dX = J^T dY of the f64 function; ``rotation_mode`` selects how the
    rotation u (and the table entries it multiplies) are rounded before the
    float64 norm gradient, as the library computes it."""
    B, T, NH, D = X.shape
    d = D // 2
    u = rotate(X, sin, cos, positions, rotation_mode).astype(np.float64)
    eps = float(EPS["bf16"] if rotation_mode == "bf16" else EPS["f32"])
    r = np.sqrt(np.sum(u * u, axis=-1, keepdims=True) / D + eps)
    y = u / r
    g = np.asarray(dY, dtype=np.float64) * 1.2
    gu = (g - y * np.sum(g * y, axis=-1, keepdims=True) / D) / r
    s, c = _columns(sin, cos, B, T, positions)
    if rotation_mode == "bf16":
        s, c = bf16_round(s), bf16_round(c)
    s, c = s.astype(np.float64), c.astype(np.float64)
    g1, g2 = gu[..., :d], gu[..., d:]
    return np.concatenate([g1 * c - g2 * s, g1 * s + g2 * c], axis=-1)
