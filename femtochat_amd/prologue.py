"""The attention prologue of femtochat's ``CausalSelfAttention``, on the MI355X.

Before calling ``attention``, the reference rotates Q and K with the rotary
embedding and RMS-normalises them over the head dimension, scaled by 1.2
(src/gpt.jl:101-106).  Here that is one memory-bound HIP kernel per tensor
that writes the result straight into the attention kernels' layout, and its
backward.

====================================================  ==========================================================
reference (Julia)                                     here (Python, torch tensors on a HIP device)
====================================================  ==========================================================
``rotary_embeddings(A, seq_len, head_dim, base)``     ``rotary_embeddings(seq_len, head_dim, base, device=)``
(src/parameters.jl:409-427)
``rotary_factors(sin_cos, positions)`` (gpt.jl:43)    ``positions=`` of the calls below (gathered in the kernel)
``apply_rotary_embedding`` + ``norm(.) .* 1.2f0``     ``attention_prologue(X, sin_cos, positions=None)``
(gpt.jl:53-77, 15-20, 103-106)                        ``attention_prologue_(Y, X, sin_cos, positions=None)``
their reverse pass (Enzyme)                           ``delta_attention_prologue_(dX, dY, X, sin_cos, ...)``
                                                      ``AttentionPrologueFunction`` (autograd)
====================================================  ==========================================================

Layout: X of Julia size (D, NH, T, B) is a torch tensor (B, T, NH, D); the
tables, Julia (D/2, L) Float32, are torch (L, D/2) float32; positions (T, B)
Int32 is a (B, T) int32 tensor.  ``sin_cos`` is the reference's
``(rope_sin, rope_cos)`` tuple.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib
from .kernels import _check_tensor, _ptr, _stream_ptr

__all__ = [
    "rotary_embeddings",
    "attention_prologue",
    "attention_prologue_",
    "delta_attention_prologue_",
    "AttentionPrologueFunction",
    "prologue_hbm_bytes",
]


def rotary_embeddings(seq_len: int, head_dim: int, base: float = 100_000.0, device=None):
    """``(sin, cos)`` tables, each (seq_len, head_dim // 2) float32:
    ``freqs[t, j] = t / base ** (2j / head_dim)`` (src/parameters.jl:409-427,
    where the channel range is ``(1:2:head_dim) .- 1`` and ``t = 0:seq_len-1``).

    The inverse frequencies are formed in float64 and rounded to float32, the
    products ``inv_freq * t`` in float32 as the reference does, and sin/cos of
    those float32 angles in float64 rounded to float32."""
    if head_dim % 2 != 0 or head_dim <= 0 or seq_len <= 0:
        raise ValueError("head_dim must be even and positive, seq_len positive")
    channel = torch.arange(0, head_dim, 2, dtype=torch.float64)
    inv_freq = (1.0 / float(base) ** (channel / head_dim)).to(torch.float32)
    t = torch.arange(seq_len, dtype=torch.float32)
    freqs = t[:, None] * inv_freq[None, :]  # float32 products
    f64 = freqs.to(torch.float64)
    sin, cos = torch.sin(f64).to(torch.float32), torch.cos(f64).to(torch.float32)
    if device is not None:
        sin, cos = sin.to(device), cos.to(device)
    return sin.contiguous(), cos.contiguous()


def _desc(X: torch.Tensor, table_len: int, overwrite: bool) -> _lib.RopeNormDesc:
    B, T, NH, D = X.shape
    d = _lib.RopeNormDesc()
    d.D, d.NH, d.T, d.B = D, NH, T, B
    d.table_len = table_len
    d.dtype = _lib.FC_BF16 if X.dtype == torch.bfloat16 else _lib.FC_F32
    d.flags = _lib.FC_FLAG_OVERWRITE if overwrite else 0
    return d


def _check(X: torch.Tensor, sin_cos, positions):
    if not isinstance(X, torch.Tensor) or X.dim() != 4:
        raise ValueError("X must be a (B, T, NH, D) tensor")
    device = X.device
    if device.type != "cuda":
        raise ValueError("the MI355X prologue needs tensors on a HIP device (torch 'cuda'); there is no CPU path")
    B, T, NH, D = X.shape
    _check_tensor("X", X, (B, T, NH, D), (torch.float32, torch.bfloat16), device)
    if len(sin_cos) != 2:
        raise ValueError("sin_cos must be the (sin, cos) pair of rotary_embeddings")
    sin, cos = sin_cos
    if sin.dim() != 2 or sin.shape[1] != D // 2:
        raise ValueError(f"the tables must be (L, {D // 2}) for head_dim {D}")
    L = sin.shape[0]
    _check_tensor("sin", sin, (L, D // 2), (torch.float32,), device)
    _check_tensor("cos", cos, (L, D // 2), (torch.float32,), device)
    if positions is not None:
        _check_tensor("positions", positions, (B, T), (torch.int32,), device)
    return device, L


def attention_prologue_(Y: torch.Tensor, X: torch.Tensor, sin_cos, positions: Optional[torch.Tensor] = None) -> None:
    """Y = norm(apply_rotary_embedding(X)) * 1.2 into a caller buffer
    (src/gpt.jl:103-106 for one tensor), in X's precision (float32, or
    bfloat16 rounded after each operation as Julia's BFloat16 is)."""
    device, L = _check(X, sin_cos, positions)
    _check_tensor("Y", Y, tuple(X.shape), (X.dtype,), device)
    sin, cos = sin_cos
    d = _desc(X, L, overwrite=True)
    _lib.check(_lib.lib().fc_rope_norm_fwd(ctypes.byref(d), _ptr(X), _ptr(sin), _ptr(cos), _ptr(positions), _ptr(Y),
                                           _stream_ptr(device)))


def attention_prologue(X: torch.Tensor, sin_cos, positions: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The rotated, normalised, 1.2-scaled tensor (new allocation)."""
    Y = torch.empty_like(X)
    attention_prologue_(Y, X, sin_cos, positions)
    return Y


def delta_attention_prologue_(dX: torch.Tensor, dY: torch.Tensor, X: torch.Tensor, sin_cos,
                              positions: Optional[torch.Tensor] = None, *, accumulate: bool = True) -> None:
    """Reverse of the prologue: dX += J^T dY (dX = J^T dY with
    ``accumulate=False``), recomputing the rotation and the norm from X; the
    gradient of the exact function in float32 at the rounded rotation."""
    device, L = _check(X, sin_cos, positions)
    _check_tensor("dY", dY, tuple(X.shape), (X.dtype,), device)
    _check_tensor("dX", dX, tuple(X.shape), (X.dtype,), device)
    sin, cos = sin_cos
    d = _desc(X, L, overwrite=not accumulate)
    _lib.check(_lib.lib().fc_rope_norm_bwd(ctypes.byref(d), _ptr(dY), _ptr(X), _ptr(sin), _ptr(cos), _ptr(positions),
                                           _ptr(dX), _stream_ptr(device)))


class AttentionPrologueFunction(torch.autograd.Function):
    """``AttentionPrologueFunction.apply(X, sin, cos, positions)``: the prologue
    as an autograd node (the tables and positions get no gradient)."""

    @staticmethod
    def forward(ctx, X, sin, cos, positions=None):
        X = X.contiguous()
        ctx.save_for_backward(X, sin, cos, positions if positions is not None else torch.empty(0))
        ctx.has_positions = positions is not None
        return attention_prologue(X, (sin, cos), positions)

    @staticmethod
    def backward(ctx, dY):
        X, sin, cos, pos = ctx.saved_tensors
        dX = torch.empty_like(X)
        delta_attention_prologue_(dX, dY.contiguous().to(X.dtype), X, (sin, cos),
                                  pos if ctx.has_positions else None, accumulate=False)
        return dX, None, None, None


def prologue_hbm_bytes(X: torch.Tensor, backward: bool = False, accumulate: bool = False) -> int:
    """Algorithmic HBM bytes of one launch: X read and Y written (forward); dY
    and X read, dX written (and read when accumulating) (backward).  The
    tables are small and L2-resident."""
    n = X.numel() * X.element_size()
    return n * ((3 + (1 if accumulate else 0)) if backward else 2)

