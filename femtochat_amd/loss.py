"""femtochat's loss-side kernels on the MI355X: cross-entropy over the
vocabulary and the token embedding, forward and gradient.

====================================================  ==========================================================
reference (Julia)                                     here (Python, torch tensors on a HIP device)
====================================================  ==========================================================
``cross_entropy(logits, targets; ignore_index,        ``cross_entropy(logits, targets, ignore_index=-1,
reduction)`` (src/gpt.jl:172-195, CUDAExt:44-50)      reduction="mean")``
``cross_entropy_gradient!(δ, logits, targets, dy,     ``cross_entropy_gradient_(delta, logits, targets, dy,
ignore_index, reduction)`` (src/kernels.jl:16-28)     ignore_index=-1, reduction="mean")``
``(𝔼::Embedding)(tokens)`` (src/gpt.jl:34)            ``embedding(weights, tokens, out_dtype=None)``
``embedding_gradient!(δ, dy, tokens)``                ``embedding_gradient_(dweights, dy, tokens)``
(src/kernels.jl:8-14)
their Enzyme/Mooncake rules                           ``CrossEntropyFunction``, ``EmbeddingFunction`` (autograd)
====================================================  ==========================================================

Layout: Julia logits (V, T, B) are a torch (B, T, V) tensor (any leading
shape: the last dimension is the vocabulary), targets (B, T); embedding
weights (D, vocab) are torch (vocab, D), the output (B, T, D).  Targets and
tokens are zero-based here (``index_base=1`` takes Julia's 1-based values).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib
from .kernels import _check_tensor, _ptr, _stream_ptr

__all__ = [
    "cross_entropy",
    "cross_entropy_",
    "cross_entropy_gradient_",
    "cross_entropy_fused_",
    "valid_target_count",
    "CrossEntropyFunction",
    "embedding",
    "embedding_",
    "embedding_gradient_",
    "embedding_gradient_workspace_bytes",
    "EmbeddingFunction",
]

_REDUCTIONS = {"none": _lib.FC_REDUCE_NONE, "sum": _lib.FC_REDUCE_SUM, "mean": _lib.FC_REDUCE_MEAN}
_INDEX = {torch.int32: _lib.FC_INDEX_I32, torch.int64: _lib.FC_INDEX_I64}


def _device(t: torch.Tensor) -> torch.device:
    if t.device.type != "cuda":
        raise ValueError("the MI355X loss kernels need tensors on a HIP device (torch 'cuda'); there is no CPU path")
    return t.device


def _xent_desc(logits, targets, ignore_index, reduction, index_base, overwrite=False) -> _lib.XentDesc:
    if reduction not in _REDUCTIONS:
        raise ValueError(f"reduction must be one of {tuple(_REDUCTIONS)}, got {reduction!r}")
    if logits.dim() < 1 or tuple(targets.shape) != tuple(logits.shape[:-1]):
        raise ValueError(f"targets {tuple(targets.shape)} must have logits' leading shape {tuple(logits.shape[:-1])}")
    dev = _device(logits)
    _check_tensor("logits", logits, tuple(logits.shape), (torch.float32,), dev)
    _check_tensor("targets", targets, tuple(targets.shape), tuple(_INDEX), dev)
    d = _lib.XentDesc()
    d.V = logits.shape[-1]
    d.N = targets.numel()
    d.index_base = index_base
    d.ignore_index = ignore_index
    d.index_type = _INDEX[targets.dtype]
    d.reduction = _REDUCTIONS[reduction]
    d.flags = _lib.FC_FLAG_OVERWRITE if overwrite else 0
    return d


def cross_entropy_(losses: torch.Tensor, logits: torch.Tensor, targets: torch.Tensor, ignore_index: int = -1,
                   reduction: str = "mean", *, index_base: int = 0, lse: Optional[torch.Tensor] = None,
                   reduced: Optional[torch.Tensor] = None, count: Optional[torch.Tensor] = None) -> None:
    """Per-token losses into ``losses`` (targets' shape, float32), and on
    request the per-token log-sum-exp (``lse``), the reduced value
    (``reduced``, 1 float: sum or mean) and the valid-target count (``count``)."""
    d = _xent_desc(logits, targets, ignore_index, reduction, index_base)
    dev = logits.device
    _check_tensor("losses", losses, tuple(targets.shape), (torch.float32,), dev)
    if lse is not None:
        _check_tensor("lse", lse, tuple(targets.shape), (torch.float32,), dev)
    for name, t in (("reduced", reduced), ("count", count)):
        if t is not None:
            _check_tensor(name, t, (1,), (torch.float32,), dev)
    _lib.check(_lib.lib().fc_cross_entropy_fwd(ctypes.byref(d), _ptr(logits), _ptr(targets), _ptr(losses), _ptr(lse),
                                               _ptr(reduced), _ptr(count), _stream_ptr(dev)))


def cross_entropy(logits: torch.Tensor, targets: torch.Tensor, ignore_index: int = -1, reduction: str = "mean", *,
                  index_base: int = 0) -> torch.Tensor:
    """The losses (reduction "none", targets' shape) or the sum / mean over
    valid targets (a 0-d tensor), as src/gpt.jl:175-195."""
    losses = torch.empty(targets.shape, dtype=torch.float32, device=logits.device)
    if reduction == "none":
        cross_entropy_(losses, logits, targets, ignore_index, reduction, index_base=index_base)
        return losses
    reduced = torch.empty(1, dtype=torch.float32, device=logits.device)
    cross_entropy_(losses, logits, targets, ignore_index, reduction, index_base=index_base, reduced=reduced)
    return reduced[0]


def valid_target_count(targets: torch.Tensor, ignore_index: int = -1) -> torch.Tensor:
    """Number of targets that are not ``ignore_index`` (1 float, on the device)."""
    dev = _device(targets)
    _check_tensor("targets", targets, tuple(targets.shape), tuple(_INDEX), dev)
    d = _lib.XentDesc()
    d.V, d.N, d.index_base, d.ignore_index = 1, targets.numel(), 0, ignore_index
    d.index_type, d.reduction, d.flags = _INDEX[targets.dtype], _lib.FC_REDUCE_SUM, 0
    count = torch.empty(1, dtype=torch.float32, device=dev)
    _lib.check(_lib.lib().fc_cross_entropy_count(ctypes.byref(d), _ptr(targets), _ptr(count), _stream_ptr(dev)))
    return count


def cross_entropy_gradient_(delta: torch.Tensor, logits: torch.Tensor, targets: torch.Tensor, dy, ignore_index: int = -1,
                            reduction: str = "mean", *, index_base: int = 0, lse: Optional[torch.Tensor] = None,
                            count: Optional[torch.Tensor] = None, accumulate: bool = True) -> None:
    """delta += scale (softmax(logits) - onehot(targets)) over valid targets
    (src/kernels.jl:16-28); ``accumulate=False`` writes instead.  ``dy`` is a
    number or a device tensor (1 value for "sum"/"mean", targets' shape for
    "none"); ``lse`` (the forward's) saves a pass over the logits; ``count``
    is counted on the device when not given for "mean"."""
    d = _xent_desc(logits, targets, ignore_index, reduction, index_base, overwrite=not accumulate)
    dev = logits.device
    _check_tensor("delta", delta, tuple(logits.shape), (torch.float32,), dev)
    if not isinstance(dy, torch.Tensor):
        dy = torch.full((1,), float(dy), dtype=torch.float32, device=dev)
    dy = dy.to(device=dev, dtype=torch.float32).contiguous()
    need = targets.numel() if reduction == "none" else 1
    if dy.numel() != need:
        raise ValueError(f"dy must hold {need} value(s) for reduction {reduction!r}, got {dy.numel()}")
    if lse is not None:
        _check_tensor("lse", lse, tuple(targets.shape), (torch.float32,), dev)
    if reduction == "mean" and count is None:
        count = valid_target_count(targets, ignore_index)
    _lib.check(_lib.lib().fc_cross_entropy_bwd(ctypes.byref(d), _ptr(delta), _ptr(logits), _ptr(targets), _ptr(dy),
                                               _ptr(count), _ptr(lse), _stream_ptr(dev)))


def cross_entropy_fused_(losses: torch.Tensor, delta: torch.Tensor, logits: torch.Tensor, targets: torch.Tensor,
                         dy=1.0, ignore_index: int = -1, reduction: str = "mean", *, index_base: int = 0,
                         lse: Optional[torch.Tensor] = None, reduced: Optional[torch.Tensor] = None,
                         count: Optional[torch.Tensor] = None, accumulate: bool = False) -> None:
    """The losses and the gradient in one pass over the logits (the loss as
    the step's last node): ``cross_entropy_`` then ``cross_entropy_gradient_``
    with the logits read once.  Needs a vocabulary that is a multiple of 4 and
    at most 32768 (the library raises FC_ERR_UNSUPPORTED otherwise)."""
    d = _xent_desc(logits, targets, ignore_index, reduction, index_base, overwrite=not accumulate)
    dev = logits.device
    _check_tensor("losses", losses, tuple(targets.shape), (torch.float32,), dev)
    _check_tensor("delta", delta, tuple(logits.shape), (torch.float32,), dev)
    if not isinstance(dy, torch.Tensor):
        dy = torch.full((1,), float(dy), dtype=torch.float32, device=dev)
    dy = dy.to(device=dev, dtype=torch.float32).contiguous()
    if dy.numel() != (targets.numel() if reduction == "none" else 1):
        raise ValueError(f"dy has the wrong number of values for reduction {reduction!r}")
    for name, t, shape in (("lse", lse, tuple(targets.shape)), ("reduced", reduced, (1,)), ("count", count, (1,))):
        if t is not None:
            _check_tensor(name, t, shape, (torch.float32,), dev)
    if reduction == "mean" and count is None:
        count = valid_target_count(targets, ignore_index)
    _lib.check(_lib.lib().fc_cross_entropy_fused(ctypes.byref(d), _ptr(logits), _ptr(targets), _ptr(losses), _ptr(lse),
                                                 _ptr(reduced), _ptr(delta), _ptr(dy), _ptr(count), _stream_ptr(dev)))


class CrossEntropyFunction(torch.autograd.Function):
    """``CrossEntropyFunction.apply(logits, targets, ignore_index, reduction)``
    with the gradient kernel in the backward (the forward's log-sum-exp and
    valid count are reused)."""

    @staticmethod
    def forward(ctx, logits, targets, ignore_index=-1, reduction="mean"):
        logits = logits.contiguous()
        dev = logits.device
        losses = torch.empty(targets.shape, dtype=torch.float32, device=dev)
        lse = torch.empty(targets.shape, dtype=torch.float32, device=dev)
        reduced = torch.empty(1, dtype=torch.float32, device=dev)
        count = torch.empty(1, dtype=torch.float32, device=dev)
        cross_entropy_(losses, logits, targets, ignore_index, reduction, lse=lse, reduced=reduced, count=count)
        ctx.save_for_backward(logits, targets, lse, count)
        ctx.ignore_index, ctx.reduction = ignore_index, reduction
        return losses if reduction == "none" else reduced[0]

    @staticmethod
    def backward(ctx, dout):
        logits, targets, lse, count = ctx.saved_tensors
        delta = torch.empty_like(logits)
        dy = dout.reshape(-1) if ctx.reduction != "none" else dout
        cross_entropy_gradient_(delta, logits, targets, dy.contiguous(), ctx.ignore_index, ctx.reduction, lse=lse,
                                count=count, accumulate=False)
        # ignored targets' columns are not written by the kernel: zero them
        mask = targets == ctx.ignore_index
        if bool(mask.any()):
            delta[mask] = 0
        return delta, None, None, None


def _embed_desc(weights, tokens, y_dtype, index_base) -> _lib.EmbedDesc:
    dev = _device(weights)
    if weights.dim() != 2:
        raise ValueError("weights must be (vocab, D)")
    _check_tensor("weights", weights, tuple(weights.shape), (torch.float32,), dev)
    _check_tensor("tokens", tokens, tuple(tokens.shape), tuple(_INDEX), dev)
    d = _lib.EmbedDesc()
    d.vocab, d.D = weights.shape
    d.N = tokens.numel()
    d.index_base = index_base
    d.index_type = _INDEX[tokens.dtype]
    d.y_dtype = _lib.FC_BF16 if y_dtype == torch.bfloat16 else _lib.FC_F32
    d.flags = 0
    return d


def embedding_(y: torch.Tensor, weights: torch.Tensor, tokens: torch.Tensor, *, index_base: int = 0) -> None:
    """y[..., :] = weights[tokens[...], :] in y's dtype (float32 or bfloat16)."""
    d = _embed_desc(weights, tokens, y.dtype, index_base)
    _check_tensor("y", y, tuple(tokens.shape) + (weights.shape[1],), (torch.float32, torch.bfloat16), weights.device)
    _lib.check(_lib.lib().fc_embedding_fwd(ctypes.byref(d), _ptr(weights), _ptr(tokens), _ptr(y),
                                           _stream_ptr(weights.device)))


def embedding(weights: torch.Tensor, tokens: torch.Tensor, out_dtype: Optional[torch.dtype] = None, *,
              index_base: int = 0) -> torch.Tensor:
    """The embedding columns of the tokens (src/gpt.jl:34), converted to
    ``out_dtype`` (the model's compute type, src/gpt.jl:137) if given."""
    y = torch.empty(tuple(tokens.shape) + (weights.shape[1],), dtype=out_dtype or torch.float32, device=weights.device)
    embedding_(y, weights, tokens, index_base=index_base)
    return y


def embedding_gradient_workspace_bytes(dweights: torch.Tensor, tokens: torch.Tensor, dy_dtype=torch.float32) -> int:
    """Workspace bytes of ``embedding_gradient_(..., deterministic=True)``."""
    d = _embed_desc(dweights, tokens, dy_dtype, 0)
    n = ctypes.c_size_t(0)
    _lib.check(_lib.lib().fc_embedding_bwd_workspace_bytes(ctypes.byref(d), ctypes.byref(n)))
    return n.value


def embedding_gradient_(dweights: torch.Tensor, dy: torch.Tensor, tokens: torch.Tensor, *, index_base: int = 0,
                        deterministic: bool = False, workspace: Optional[torch.Tensor] = None) -> None:
    """dweights[tokens[t], :] += dy[t, :] (src/kernels.jl:8-14): fp32 atomics
    (the reference's order-free adds), or with ``deterministic=True`` a sort
    by id and one in-order sum per id (the same bits on every call; the
    workspace, uint8 of ``embedding_gradient_workspace_bytes`` bytes, is
    allocated here when not given)."""
    d = _embed_desc(dweights, tokens, dy.dtype, index_base)
    _check_tensor("dy", dy, tuple(tokens.shape) + (dweights.shape[1],), (torch.float32, torch.bfloat16), dweights.device)
    if not deterministic:
        _lib.check(_lib.lib().fc_embedding_bwd(ctypes.byref(d), _ptr(dweights), _ptr(dy), _ptr(tokens),
                                               _stream_ptr(dweights.device)))
        return
    n = ctypes.c_size_t(0)
    _lib.check(_lib.lib().fc_embedding_bwd_workspace_bytes(ctypes.byref(d), ctypes.byref(n)))
    if workspace is None:
        workspace = torch.empty(n.value, dtype=torch.uint8, device=dweights.device)
    _lib.check(_lib.lib().fc_embedding_bwd_sorted(ctypes.byref(d), _ptr(dweights), _ptr(dy), _ptr(tokens),
                                                  _ptr(workspace), workspace.numel(), _stream_ptr(dweights.device)))


class EmbeddingFunction(torch.autograd.Function):
    """``EmbeddingFunction.apply(weights, tokens, out_dtype)``: the embedding
    as an autograd node (the tokens get no gradient)."""

    @staticmethod
    def forward(ctx, weights, tokens, out_dtype=None):
        ctx.save_for_backward(tokens)
        ctx.vocab_shape = tuple(weights.shape)
        return embedding(weights.contiguous(), tokens, out_dtype)

    @staticmethod
    def backward(ctx, dy):
        (tokens,) = ctx.saved_tensors
        dw = torch.zeros(ctx.vocab_shape, dtype=torch.float32, device=dy.device)
        embedding_gradient_(dw, dy.contiguous(), tokens)
        return dw, None, None
