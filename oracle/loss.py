"""Restatement of femtochat's loss-side kernels (the parity oracle for them).

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import this package, and only as the checker;
the product path (femtochat_amd) never calls it.

What is restated (citations into msjgriffiths/femtochat):

* ``cross_entropy``          : ``cross_entropy(logits, targets, ignore_index,
  reduction)`` (src/gpt.jl:175-195) and its CUDA kernel
  (ext/FemtoChatCUDAExt.jl:21-54): per token, loss = max + log(sum(exp(x -
  max))) - x[target], zero where target == ignore_index; reduction "none"
  (per-token losses), "sum", or "mean" (sum / number of valid targets).
* ``cross_entropy_gradient`` : ``cross_entropy_gradient!`` (src/kernels.jl:16-28,
  CUDAExt:56-61): delta += valid ? scale * (softmax(x) - onehot(target)) : 0,
  scale = dy / count(valid) ("mean"), dy ("sum"), dy[token] ("none").
* ``embedding``              : ``(E::Embedding)(tokens) = E.E[:, tokens]``
  (src/gpt.jl:34; CUDAExt:63-76), a gather of weight columns.
* ``embedding_gradient``     : ``embedding_gradient!`` (src/kernels.jl:8-14,
  CUDAExt:78-94): delta[:, tokens[t]] += dy[:, t].
* ``embedding_gradient_in_order_f32``: the same sums in one fixed float32
  order (per id, token order, zero values skipped, added once), the order of
  the library's deterministic gradient; pinned against ``embedding_gradient``
  within float32 rounding, a column receiving only zeros keeping its bits,
  and a cancellation that only that order gives.

Layout (torch, row-major): logits (N, V) with N tokens (the reference's
(V, T, B) column-major array), targets (N,), embedding weights (vocab, D)
(the reference's (D, vocab)), output (N, D).  Target and token values are
given with an index base (1 for the reference's Julia indices, 0 for
torch's); a value outside [base, base + V) other than ignore_index is not
valid input.  Arithmetic in float64.

Pinning (tests/test_loss_oracle.py): torch.nn.functional.cross_entropy and
embedding with their autograd gradients (float64), central finite
differences, closed forms (all-equal logits give log V; gradient rows sum to
zero), and planted mistakes that must fail.
"""
from __future__ import annotations

import numpy as np

REDUCTIONS = ("none", "sum", "mean")


def _valid(targets, ignore_index):
    t = np.asarray(targets).astype(np.int64)
    return t, t != ignore_index


def token_lse(logits) -> np.ndarray:
    """log(sum(exp(x))) per token, computed as max + log(sum(exp(x - max)))."""
    x = np.asarray(logits, dtype=np.float64)
    m = np.max(x, axis=-1)
    return m + np.log(np.sum(np.exp(x - m[:, None]), axis=-1))


def cross_entropy(logits, targets, ignore_index: int = -1, reduction: str = "mean", base: int = 1):
    """Losses (reduction "none") or the reduced scalar, float64."""
    if reduction not in REDUCTIONS:
        raise ValueError(reduction)
    x = np.asarray(logits, dtype=np.float64)
    t, valid = _valid(targets, ignore_index)
    idx = np.where(valid, t - base, 0)
    losses = np.where(valid, token_lse(x) - x[np.arange(x.shape[0]), idx], 0.0)
    if reduction == "none":
        return losses
    total = float(np.sum(losses))
    return total / float(np.sum(valid)) if reduction == "mean" else total


def cross_entropy_gradient(delta, logits, targets, dy, ignore_index: int = -1, reduction: str = "mean",
                           base: int = 1) -> np.ndarray:
    """delta + d(loss)/d(logits) scaled by dy (a new float64 array)."""
    x = np.asarray(logits, dtype=np.float64)
    N, V = x.shape
    t, valid = _valid(targets, ignore_index)
    if reduction == "none":
        scale = np.asarray(dy, dtype=np.float64).reshape(N)
    elif reduction == "mean":
        scale = np.full(N, float(dy) / float(np.sum(valid)))
    else:
        scale = np.full(N, float(dy))
    p = np.exp(x - token_lse(x)[:, None])
    onehot = np.zeros_like(p)
    onehot[np.arange(N)[valid], (t - base)[valid]] = 1.0
    g = np.where(valid[:, None], scale[:, None] * (p - onehot), 0.0)
    return np.asarray(delta, dtype=np.float64) + g


def embedding(weights, tokens, base: int = 1) -> np.ndarray:
    """Rows of the (vocab, D) weights selected by the tokens: (N, D)."""
    w = np.asarray(weights)
    return w[np.asarray(tokens).astype(np.int64) - base]


def embedding_gradient(delta, dy, tokens, base: int = 1) -> np.ndarray:
    """delta with dy's rows added at the tokens' rows (repeats accumulate)."""
    out = np.array(delta, dtype=np.float64, copy=True)
    np.add.at(out, np.asarray(tokens).astype(np.int64) - base, np.asarray(dy, dtype=np.float64))
    return out


def embedding_gradient_in_order_f32(delta, dy, tokens, base: int = 1) -> np.ndarray:
    """The same gradient in one fixed float32 order: per id, its dy rows summed
    in token order (zero values skipped, from -0), the sum added to delta once;
    ids outside the table add nothing.  The reference's atomic adds
    (CUDAExt:78-94) have no order; this is the order of the library's
    deterministic gradient, whose bits it must match.  Its sums equal
    embedding_gradient's within float32 rounding."""
    out = np.array(delta, dtype=np.float32, copy=True)
    ids = np.asarray(tokens).astype(np.int64) - base
    dy = np.asarray(dy, dtype=np.float32)
    order = np.argsort(ids, kind="stable")
    sorted_ids = ids[order]
    heads = np.flatnonzero(np.r_[True, sorted_ids[1:] != sorted_ids[:-1]])
    ends = np.r_[heads[1:], len(ids)]
    for h, e in zip(heads, ends):
        i = sorted_ids[h]
        if i < 0 or i >= out.shape[0]:
            continue
        s = np.full(out.shape[1], -0.0, np.float32)
        for t in order[h:e]:
            v = dy[t]
            s = np.where(v != 0, (s + v).astype(np.float32), s)
        out[i] = (out[i] + s).astype(np.float32)
    return out
