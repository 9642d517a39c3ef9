"""GPU parity of the loss-side kernels (cross-entropy, embedding) against
oracle/loss.py, through the C ABI (femtochat_amd.loss).

Cross-entropy is fp32 arithmetic in both the reference and here: losses,
log-sum-exp and gradients are compared with the float64 oracle within 1e-5
(relative to the tensor's largest magnitude).  The embedding gather is a
copy and must be bit-exact (bf16 output: torch's float32 -> bfloat16
conversion); the scatter-add gradient sums repeated tokens with atomics in an
unspecified order, so it is compared within 1e-5, and exactly where every
token is distinct.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from femtochat_amd import (CrossEntropyFunction, EmbeddingFunction, cross_entropy, cross_entropy_,
                           cross_entropy_fused_, cross_entropy_gradient_, embedding, embedding_gradient_,
                           valid_target_count)
from femtochat_amd import _lib
from oracle import loss as O

from tests.helpers import rel_err, say

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _ce_case(gpu, N, V, seed, ignore_frac=0.25, scale=3.0, dtype=torch.int32, base=0, shift=0.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, V, generator=g) * scale + shift
    t = torch.randint(0, V, (N,), generator=g) + base
    t[torch.rand(N, generator=g) < ignore_frac] = -1
    return x, t.to(dtype), x.to(gpu), t.to(dtype).to(gpu)


@pytest.mark.parametrize("V", [1, 53, 1000, 4096])
@pytest.mark.parametrize("reduction", ["none", "sum", "mean"])
def test_cross_entropy_matches_oracle(gpu, V, reduction):
    x, t, xd, td = _ce_case(gpu, 67, V, seed=V)
    got = cross_entropy(xd, td, -1, reduction)
    ref = O.cross_entropy(x.numpy(), t.numpy(), -1, reduction, base=0)
    if reduction == "none":
        assert rel_err(got.cpu().numpy(), ref) < TOL
    else:
        assert abs(float(got) - ref) <= TOL * max(abs(ref), 1.0)


@pytest.mark.parametrize("dtype,base", [(torch.int64, 1), (torch.int32, 1), (torch.int64, 0)])
def test_index_types_and_bases(gpu, dtype, base):
    x, t, xd, td = _ce_case(gpu, 40, 300, seed=5, dtype=dtype, base=base)
    losses = torch.empty(40, device=gpu)
    lse = torch.empty(40, device=gpu)
    count = torch.empty(1, device=gpu)
    cross_entropy_(losses, xd, td, -1, "mean", index_base=base, lse=lse, count=count)
    assert rel_err(losses.cpu().numpy(), O.cross_entropy(x.numpy(), t.numpy(), -1, "none", base=base)) < TOL
    assert np.max(np.abs(lse.cpu().numpy() - O.token_lse(x.numpy()))) < TOL
    assert float(count) == float((t != -1).sum())


def test_large_logits_and_bad_targets(gpu):
    x, t, xd, td = _ce_case(gpu, 30, 512, seed=6, ignore_frac=0.0, shift=1e4)
    got = cross_entropy(xd, td, -1, "none").cpu().numpy()
    np.testing.assert_allclose(got, O.cross_entropy(x.numpy(), t.numpy(), -1, "none", 0), rtol=0, atol=2e-3)
    # (fp32 logits near 1e4 carry 1e-3 of rounding themselves)
    bad = td.clone()
    bad[3] = 512
    bad[4] = -7
    out = cross_entropy(xd, bad, -1, "none").cpu().numpy()
    assert np.isnan(out[[3, 4]]).all() and np.isfinite(np.delete(out, [3, 4])).all()
    none_valid = torch.full_like(td, -1)
    assert np.isnan(float(cross_entropy(xd, none_valid, -1, "mean")))  # 0 / 0, as the reference
    assert float(cross_entropy(xd, none_valid, -1, "sum")) == 0.0


@pytest.mark.parametrize("V", [53, 4096])
@pytest.mark.parametrize("reduction", ["none", "sum", "mean"])
@pytest.mark.parametrize("with_lse", [False, True])
def test_gradient_matches_oracle(gpu, V, reduction, with_lse):
    x, t, xd, td = _ce_case(gpu, 45, V, seed=100 + V)
    g = torch.Generator().manual_seed(9)
    dy = torch.randn(45, generator=g) if reduction == "none" else torch.tensor([0.37])
    base = torch.randn(45, V, generator=g)
    delta = base.to(gpu)
    lse = None
    if with_lse:
        lse = torch.empty(45, device=gpu)
        cross_entropy_(torch.empty(45, device=gpu), xd, td, -1, reduction, lse=lse)
    cross_entropy_gradient_(delta, xd, td, dy.to(gpu), -1, reduction, lse=lse)
    d = delta.cpu().numpy()
    ref = O.cross_entropy_gradient(base.numpy(), x.numpy(), t.numpy(),
                                   dy.numpy() if reduction == "none" else float(dy), -1, reduction, base=0)
    # accumulating is an fp32 addition onto delta (as the reference's `+=`):
    # within 1e-5 of the gradient plus that addition's rounding
    gref = ref - base.numpy()
    bound = TOL * np.max(np.abs(gref)) + 2.0 ** -23 * np.abs(ref)
    assert np.all(np.abs(d - ref) <= bound)
    # ignored columns are untouched, bit for bit
    ign = (t == -1).numpy()
    assert np.array_equal(d[ign], base.numpy()[ign])
    # overwrite writes the gradient itself
    delta2 = base.to(gpu)
    cross_entropy_gradient_(delta2, xd, td, dy.to(gpu), -1, reduction, lse=lse, accumulate=False)
    keep = ~ign
    assert rel_err(delta2.cpu().numpy()[keep], (ref - base.numpy())[keep]) < TOL


@pytest.mark.parametrize("V", [4, 4096, 32768])
@pytest.mark.parametrize("reduction", ["none", "mean"])
@pytest.mark.parametrize("accumulate", [False, True])
def test_fused_matches_oracle(gpu, V, reduction, accumulate):
    N = 37
    x, t, xd, td = _ce_case(gpu, N, V, seed=300 + V)
    g = torch.Generator().manual_seed(10)
    dy = torch.randn(N, generator=g) if reduction == "none" else torch.tensor([0.9])
    base = torch.randn(N, V, generator=g)
    delta = base.to(gpu)
    losses, lse, reduced = torch.empty(N, device=gpu), torch.empty(N, device=gpu), torch.empty(1, device=gpu)
    cross_entropy_fused_(losses, delta, xd, td, dy.to(gpu), -1, reduction, lse=lse, reduced=reduced,
                         accumulate=accumulate)
    assert rel_err(losses.cpu().numpy(), O.cross_entropy(x.numpy(), t.numpy(), -1, "none", 0)) < TOL
    assert np.max(np.abs(lse.cpu().numpy() - O.token_lse(x.numpy()))) < TOL
    if reduction == "mean":
        assert abs(float(reduced) - O.cross_entropy(x.numpy(), t.numpy(), -1, "mean", 0)) < TOL
    gref = O.cross_entropy_gradient(np.zeros((N, V)), x.numpy(), t.numpy(),
                                    dy.numpy() if reduction == "none" else float(dy), -1, reduction, 0)
    d = delta.cpu().numpy()
    keep = (t != -1).numpy()
    if accumulate:
        ref = base.numpy() + gref
        assert np.all(np.abs(d - ref) <= TOL * np.max(np.abs(gref)) + 2.0 ** -23 * np.abs(ref))
    else:
        assert rel_err(d[keep], gref[keep]) < TOL
    assert np.array_equal(d[~keep], base.numpy()[~keep])  # ignored columns untouched


def test_fused_keeps_a_caller_count(gpu):
    # A count normalised over several micro-batches (here 3x the local one)
    # scales the gradient and is left as the caller passed it; the reduced
    # mean is the local one, as cross_entropy_ reports it.
    N, V = 29, 4096
    x, t, xd, td = _ce_case(gpu, N, V, seed=77)
    local = float((t != -1).sum())
    count = torch.tensor([3.0 * local], device=gpu)
    losses, reduced = torch.empty(N, device=gpu), torch.empty(1, device=gpu)
    delta = torch.zeros(N, V, device=gpu)
    cross_entropy_fused_(losses, delta, xd, td, 1.0, -1, "mean", reduced=reduced, count=count)
    torch.cuda.synchronize()
    assert float(count) == 3.0 * local
    assert abs(float(reduced) - O.cross_entropy(x.numpy(), t.numpy(), -1, "mean", 0)) < TOL
    gref = O.cross_entropy_gradient(np.zeros((N, V)), x.numpy(), t.numpy(), 1.0, -1, "mean", 0) / 3.0
    keep = (t != -1).numpy()
    assert rel_err(delta.cpu().numpy()[keep], gref[keep]) < TOL


def test_fused_rejects_what_it_cannot_hold(gpu):
    x, t, xd, td = _ce_case(gpu, 4, 53, seed=1)
    with pytest.raises(_lib.AttentionError, match="multiple of 4"):
        cross_entropy_fused_(torch.empty(4, device=gpu), torch.zeros_like(xd), xd, td, 1.0, -1, "sum")
    x = torch.zeros(2, 32772, device=gpu)
    with pytest.raises(_lib.AttentionError, match="32768"):
        cross_entropy_fused_(torch.empty(2, device=gpu), torch.zeros_like(x), x, torch.zeros(2, dtype=torch.int32,
                                                                                               device=gpu), 1.0)


def test_autograd_cross_entropy(gpu):
    x, t, xd, td = _ce_case(gpu, 33, 777, seed=11)
    xg = xd.clone().requires_grad_(True)
    loss = CrossEntropyFunction.apply(xg, td, -1, "mean")
    loss.backward()
    x64 = x.double().requires_grad_(True)
    ref = F.cross_entropy(x64, t.long(), ignore_index=-1, reduction="mean")
    ref.backward()
    assert abs(float(loss) - float(ref)) < TOL
    assert rel_err(xg.grad.cpu().numpy(), x64.grad.numpy()) < TOL
    assert float(valid_target_count(td)) == float((t != -1).sum())


def test_cross_entropy_bench_size_properties(gpu):
    # The training-step shape (vocabulary 2^15, 4 x 2048 tokens): equal logits
    # give log V per token and gradient columns summing to zero; random logits
    # match the oracle on the first and last tokens.
    N, V = 8192, 32768
    say(f"cross-entropy full size: N={N} V={V}")
    x = torch.full((N, V), 0.25, device=gpu)
    t = torch.randint(0, V, (N,), device=gpu, dtype=torch.int32)
    losses = cross_entropy(x, t, -1, "none")
    assert float((losses - float(np.log(V))).abs().max()) < 2e-6
    g = torch.Generator(device=gpu).manual_seed(3)
    x = torch.randn(N, V, device=gpu, generator=g) * 4
    t[::7] = -1
    lse = torch.empty(N, device=gpu)
    losses = torch.empty(N, device=gpu)
    cross_entropy_(losses, x, t, -1, "mean", lse=lse)
    delta = torch.zeros(N, V, device=gpu)
    cross_entropy_gradient_(delta, x, t, 1.0, -1, "sum", lse=lse)
    assert float(delta.double().sum(dim=1).abs().max()) < 1e-5
    for rows in (slice(0, 16), slice(N - 16, N)):
        xs, ts = x[rows].cpu().numpy(), t[rows].cpu().numpy()
        assert rel_err(losses[rows].cpu().numpy(), O.cross_entropy(xs, ts, -1, "none", 0)) < TOL
        ref = O.cross_entropy_gradient(np.zeros_like(xs), xs, ts, 1.0, -1, "sum", 0)
        assert rel_err(delta[rows].cpu().numpy(), ref) < TOL


# ---- embedding -------------------------------------------------------------------
@pytest.mark.parametrize("D", [13, 64, 512])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_embedding_gather_is_exact(gpu, D, out):
    g = torch.Generator().manual_seed(D)
    W = torch.randn(101, D, generator=g)
    tok = torch.randint(0, 101, (5, 9), generator=g)
    y = embedding(W.to(gpu), tok.to(torch.int32).to(gpu), out).cpu()
    ref = torch.from_numpy(O.embedding(W.numpy(), tok.numpy(), base=0)).to(out)
    assert torch.equal(y, ref)


def test_embedding_bad_tokens_and_bases(gpu):
    W = torch.randn(20, 32)
    tok = torch.tensor([1, 20, 5, 0, 21, -3], dtype=torch.int64)  # 1-based: 0, 21, -3 are outside
    y = embedding(W.to(gpu), tok.to(gpu), index_base=1).cpu()
    good = [0, 1, 2]
    assert torch.equal(y[good], W[tok[good] - 1])
    assert torch.isnan(y[[3, 4, 5]]).all()
    dW = torch.zeros(20, 32, device=gpu)
    embedding_gradient_(dW, torch.ones(6, 32, device=gpu), tok.to(gpu), index_base=1)
    ref = O.embedding_gradient(np.zeros((20, 32)), np.ones((3, 32)), tok[good].numpy(), base=1)
    assert np.array_equal(dW.cpu().numpy(), ref)


@pytest.mark.parametrize("dy_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("D", [13, 512])
def test_embedding_gradient_matches_oracle(gpu, dy_dtype, D):
    g = torch.Generator().manual_seed(40 + D)
    vocab, N = 64, 300
    tok = torch.randint(0, vocab, (N,), generator=g)
    tok[:50] = 7  # a heavily repeated token
    dy = torch.randn(N, D, generator=g).to(dy_dtype)
    dy[60:70] = 0  # zero rows add nothing (skipped)
    base = torch.randn(vocab, D, generator=g)
    dW = base.to(gpu)
    embedding_gradient_(dW, dy.to(gpu), tok.to(torch.int32).to(gpu))
    ref = O.embedding_gradient(base.numpy(), dy.float().numpy(), tok.numpy(), base=0)
    assert rel_err(dW.cpu().numpy() - base.numpy(), ref - base.numpy()) < TOL
    # distinct tokens: every element receives one addition, so the result is exact
    uniq = torch.randperm(vocab, generator=g)[:40]
    dW2 = base.to(gpu)
    embedding_gradient_(dW2, dy[:40].to(gpu), uniq.to(gpu))
    exact = base.clone()
    exact[uniq] += dy[:40].float()
    assert torch.equal(dW2.cpu(), exact)


@pytest.mark.parametrize("dy_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("itype,base", [(torch.int32, 0), (torch.int64, 1)])
@pytest.mark.parametrize("D", [1, 37, 512, 600])
def test_sorted_embedding_gradient_is_bit_exact(gpu, dy_dtype, itype, base, D):
    # the deterministic gradient sums each id's rows in token order and adds
    # once: it must equal the oracle's float32 restatement of that order bit
    # for bit (repeats, zero values, signed zeros, ids outside the table)
    g = torch.Generator().manual_seed(D * 3 + base)
    vocab, N = 50, 700
    tok = torch.randint(0, vocab, (N,), generator=g)
    tok[:80] = 9                       # one heavily repeated id
    tok[100:103] = torch.tensor([-1, vocab, 3 * vocab])  # outside the table (after the base shift)
    dy = torch.randn(N, D, generator=g).to(dy_dtype)
    dy[200:220] = 0.0                  # zero values are skipped
    dy[230, : min(D, 5)] = -0.0
    delta = torch.randn(vocab, D, generator=g)
    delta[::7] = -0.0                  # a column receiving only zeros keeps its bits
    dW = delta.to(gpu)
    tokens = (tok + base).to(itype)
    embedding_gradient_(dW, dy.to(gpu), tokens.to(gpu), index_base=base, deterministic=True)
    exact = O.embedding_gradient_in_order_f32(delta.numpy(), dy.float().numpy(), tokens.numpy(), base=base)
    got = dW.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), exact.view(np.uint32))
    # and the mathematics: within float32 rounding of the float64 sums
    keep = (tok >= 0) & (tok < vocab)
    ref = O.embedding_gradient(delta.numpy(), dy.float().numpy()[keep.numpy()], tok[keep].numpy(), base=0)
    assert rel_err(got - delta.numpy(), ref - delta.numpy()) < 1e-5


def test_sorted_embedding_gradient_training_size(gpu):
    # scripts/train.jl's shape (4 x 2048 tokens, 512 wide, vocabulary 2^15):
    # the same bits on every call, the order's exact sums, and the atomic
    # gradient within float32 rounding
    g = torch.Generator().manual_seed(5)
    vocab, N, D = 32768, 8192, 512
    tok = torch.randint(0, vocab, (N,), generator=g, dtype=torch.int32)
    tok[:1000] = 17
    dy = torch.randn(N, D, generator=g)
    runs = []
    for _ in range(2):
        dW = torch.zeros(vocab, D, device=gpu)
        embedding_gradient_(dW, dy.to(gpu), tok.to(gpu), deterministic=True)
        runs.append(dW.cpu())
    assert torch.equal(runs[0], runs[1])
    exact = O.embedding_gradient_in_order_f32(np.zeros((vocab, D), np.float32), dy.numpy(), tok.numpy(), base=0)
    assert np.array_equal(runs[0].numpy().view(np.uint32), exact.view(np.uint32))
    dA = torch.zeros(vocab, D, device=gpu)
    embedding_gradient_(dA, dy.to(gpu), tok.to(gpu))
    assert torch.allclose(dA.cpu(), runs[0], rtol=1e-5, atol=1e-4)


def test_autograd_embedding(gpu):
    W = torch.randn(50, 24)
    tok = torch.randint(0, 50, (4, 11))
    Wg = W.to(gpu).requires_grad_(True)
    y = EmbeddingFunction.apply(Wg, tok.to(gpu), None)
    dy = torch.randn(4, 11, 24)
    y.backward(dy.to(gpu))
    Wc = W.clone().double().requires_grad_(True)
    F.embedding(tok, Wc).backward(dy.double())
    assert rel_err(Wg.grad.cpu().numpy(), Wc.grad.numpy()) < TOL


def test_embedding_bench_size(gpu):
    # The training-step shape: D = 512, vocabulary 2^15, 4 x 2048 tokens.
    D, vocab, N = 512, 32768, 8192
    say(f"embedding full size: D={D} vocab={vocab} N={N}")
    g = torch.Generator(device=gpu).manual_seed(5)
    W = torch.randn(vocab, D, device=gpu, generator=g)
    tok = torch.randint(0, vocab, (N,), device=gpu, generator=g, dtype=torch.int32)
    y = embedding(W, tok)
    assert torch.equal(y, W[tok.long()])
    dy = torch.randn(N, D, device=gpu, generator=g)
    dW = torch.zeros_like(W)
    embedding_gradient_(dW, dy, tok)
    ref = torch.zeros(vocab, D, device=gpu, dtype=torch.float64).index_add_(0, tok.long(), dy.double())
    assert rel_err(dW.cpu().numpy(), ref.cpu().numpy()) < TOL
