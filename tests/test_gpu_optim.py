"""GPU parity of the optimizer kernels against oracle/optim.py.

The elementwise updates (AdamW step, CUDA Adam/Muon final writes,
gather/scatter) run the reference's fp32 operations in its order without
contraction, so they must equal the float32 oracle bit for bit, on both the
16-byte path and the scalar tail.  Polar Express runs fp32 batched GEMMs
(rocBLAS) through five polynomial steps whose coefficients reach 22, which
could amplify rounding in the smallest singular directions: it is compared
with the float64 oracle and with the same iteration in plain torch fp32
within the fp32 contract's 1e-4 (measured: about 1e-5 at 512 x 2048).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from femtochat_amd import AdamW, adam_update_, gather_, muon_update_, polar_express, scatter_
from femtochat_amd.optim import polar_express_grouped_
from oracle import optim as O

from tests.helpers import rel_err, say

pytestmark = pytest.mark.gpu

# Polar Express: max |X - R| / max |R| against float64, and against torch fp32
POLAR_TOL = 1e-4
# bf16 compute type: the reference's own bf16 iteration (emulated in torch,
# below) lies 2.5-3.3e-2 from the float64 mathematics at these sizes; this one
# must stay within 4e-2 of float64 and no further from it than 1.5 times the
# emulated reference, and two bf16 runs differ by both of their roundings.
POLAR_TOL_BF16 = 4e-2


@pytest.mark.parametrize("n,misalign", [(1_000_003, 0), (4096, 1), (7, 0)])
def test_adamw_steps_are_bit_exact(gpu, n, misalign):
    g = torch.Generator().manual_seed(n)
    theta = torch.randn(n + misalign, generator=g)
    dev_theta = theta.to(gpu)[misalign:]  # misalign = 1: 4-byte offset, the scalar path
    opt = AdamW(dev_theta, alpha=0.02, beta1=0.8, beta2=0.95, eps=1e-10, lam=0.01)
    th, m, v = theta[misalign:].numpy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    for t in range(1, 5):
        grad = torch.randn(n, generator=g) * (0.1 * t)
        gbuf = torch.zeros(n + misalign)
        gbuf[misalign:] = grad
        opt(dev_theta, gbuf.to(gpu)[misalign:], grad_scale=2.0 if t == 3 else 1.0)
        th, m, v = O.adamw_step(th, grad.numpy(), m, v, t, 0.02, 0.8, 0.95, 1e-10, 0.01,
                                grad_scale=2.0 if t == 3 else 1.0)
    assert np.array_equal(dev_theta.cpu().numpy(), th)
    assert np.array_equal(opt.m.cpu().numpy(), m) and np.array_equal(opt.v.cpu().numpy(), v)


@pytest.mark.parametrize("t", [3, 10, 999, 12288])
def test_adamw_bias_corrections_at_large_step_counts(gpu, t):
    # the host forms 1 - beta^t as Julia's Float32 ^ Int does (x*x*x at t = 3,
    # square-and-multiply in Float64 otherwise); the step must stay bit-exact
    g = torch.Generator().manual_seed(t)
    n = 4099
    theta, grad = torch.randn(n, generator=g), torch.randn(n, generator=g)
    m0, v0 = torch.randn(n, generator=g) * 0.1, torch.rand(n, generator=g) * 0.01
    th = theta.to(gpu)
    opt = AdamW(th, alpha=0.004, beta1=0.8, beta2=0.96, eps=1e-10, lam=0.01, t=t - 1)
    opt.m.copy_(m0)
    opt.v.copy_(v0)
    opt(th, grad.to(gpu))
    ref, m, v = O.adamw_step(theta.numpy(), grad.numpy(), m0.numpy(), v0.numpy(), t, 0.004, 0.8, 0.96, 1e-10, 0.01)
    assert np.array_equal(th.cpu().numpy(), ref) and np.array_equal(opt.m.cpu().numpy(), m)


def test_adam_update_is_bit_exact(gpu):
    g = torch.Generator().manual_seed(1)
    Th = torch.randn(5000, generator=g)
    m, v = torch.randn(3000, generator=g), torch.rand(3000, generator=g)
    scal = [torch.tensor([x], device=gpu) for x in (0.05, 0.3, 0.01)]
    Td = Th.to(gpu)
    adam_update_(Td, 1234, m.to(gpu), v.to(gpu), *scal, lam=0.1, eps=1e-8)
    ref = O.adam_update(Th.numpy(), 1234, m.numpy(), v.numpy(), 0.05, 0.3, 0.01, 0.1, 1e-8)
    assert np.array_equal(Td.cpu().numpy(), ref)


def test_muon_update_gather_scatter_are_bit_exact(gpu):
    g = torch.Generator().manual_seed(2)
    width, count = 48 * 32, 5
    Th = torch.randn(20000, generator=g)
    Th[::17] = 0.0  # zero parameters: x * theta = 0 takes the decay branch
    offsets = torch.tensor([0, 3000, 7000, 11111, 15000], dtype=torch.int64)
    X = torch.randn(count, width, generator=g)
    X[:, ::13] = 0.0
    Td = Th.to(gpu)
    muon_update_(Td, X.to(gpu), torch.tensor([0.02], device=gpu), torch.tensor([0.1], device=gpu), offsets.to(gpu))
    ref = O.muon_update(Th.numpy(), X.numpy(), offsets.numpy(), 0.02, 0.1)
    assert np.array_equal(Td.cpu().numpy(), ref)
    stack = torch.empty(count, width, device=gpu)
    gather_(stack, Td, offsets.to(gpu))
    assert np.array_equal(stack.cpu().numpy(), O.gather(ref, offsets.numpy(), width))
    out = torch.zeros(20000, device=gpu)
    scatter_(out, stack * 2, offsets.to(gpu))
    assert np.array_equal(out.cpu().numpy(), O.scatter(np.zeros(20000, np.float32), O.gather(ref, offsets.numpy(), width) * 2,
                                                       offsets.numpy()))


def _torch_polar_f32(G):
    """The same iteration in plain torch fp32 (Julia (m, n) = torch (n, m) per matrix)."""
    out = []
    for g in G:  # g: torch (n, m) = G_j^T
        M = g.T  # (m, n)
        transposed = M.shape[0] > M.shape[1]
        X = (M.T if transposed else M) / (np.float32(1.01) * torch.sqrt((M * M).sum()) + np.float32(1e-6))
        for a, b, c in O.COEFFICIENTS:
            A = X @ X.T.contiguous()
            B = np.float32(b) * A + np.float32(c) * (A @ A)
            X = np.float32(a) * X + B @ X
        out.append((X.T if transposed else X).T)
    return torch.stack(out)


@pytest.mark.parametrize("m,n,k", [(64, 64, 3), (48, 160, 2), (160, 48, 2), (512, 2048, 1), (2048, 512, 1)])
def test_polar_express_matches_oracle(gpu, m, n, k):
    g = torch.Generator().manual_seed(m * 7 + n)
    G = torch.randn(k, n, m, generator=g)  # Julia (m, n, k)
    out = polar_express(G.to(gpu)).cpu()
    julia = G.numpy().transpose(0, 2, 1)  # [j] = Julia G[:, :, j] (m, n)
    ref = O.polar_express(julia).transpose(0, 2, 1)
    e64 = rel_err(out.numpy(), ref)
    e32 = rel_err(out.numpy(), _torch_polar_f32(G.to(gpu)).cpu().numpy())
    say(f"polar {m}x{n}x{k}: vs float64 {e64:.2e}, vs torch fp32 {e32:.2e}")
    assert e64 < POLAR_TOL and e32 < POLAR_TOL
    # the output's singular values are the composed polynomial of the normalised input's
    for j in range(k):
        s_in = np.linalg.svd(julia[j].astype(np.float64), compute_uv=False)
        scale = float(np.float32(1.01)) * np.sqrt(np.sum(julia[j].astype(np.float64) ** 2)) + float(np.float32(1e-6))
        s_out = np.linalg.svd(out[j].numpy().astype(np.float64), compute_uv=False)
        np.testing.assert_allclose(np.sort(s_out), np.sort(O.composed_polynomial(s_in / scale)), atol=POLAR_TOL * 4)


@pytest.mark.parametrize("m,n,k,compute_type", [(7, 13, 3, torch.float32), (13, 7, 2, torch.float32), (1, 5, 2, torch.float32),
                                                 (31, 45, 2, torch.bfloat16), (45, 31, 2, torch.bfloat16),
                                                 (33, 97, 1, torch.bfloat16)])
def test_polar_express_odd_sizes(gpu, m, n, k, compute_type):
    # m n not a multiple of 4: the copy into the iteration buffer takes its
    # element-wise path (the 16-byte one needs whole 16-byte groups).  bf16 at
    # a few tens of rows: below that one element's rounding, amplified by the
    # first steps' cancellations (coefficients up to 22), decides the max norm.
    g = torch.Generator().manual_seed(m * 11 + n)
    G = torch.randn(k, n, m, generator=g)
    out = polar_express(G.to(gpu), compute_type=compute_type).cpu()
    ref = O.polar_express(G.numpy().transpose(0, 2, 1)).transpose(0, 2, 1)
    e64 = rel_err(out.numpy(), ref)
    emu = (_torch_polar_f32 if compute_type == torch.float32 else _torch_polar_bf16)(G.to(gpu)).cpu().numpy()
    say(f"polar {compute_type} {m}x{n}x{k}: vs float64 {e64:.2e}, vs torch {rel_err(out.numpy(), emu):.2e}")
    if compute_type == torch.float32:
        assert e64 < POLAR_TOL and rel_err(out.numpy(), emu) < POLAR_TOL
    else:  # as the other bf16 cases: no further from float64 than the reference's own bf16 iteration allows
        e_ref = rel_err(emu, ref)
        assert e64 <= max(POLAR_TOL_BF16, 1.5 * e_ref)


def _torch_polar_bf16(G):
    """The reference's bf16 iteration in plain torch: bf16 buffers, fp32 scalars
    and elementwise arithmetic, products rounded to bf16."""
    out = []
    for g in G:
        M = g.T
        transposed = M.shape[0] > M.shape[1]
        X = ((M.T if transposed else M) / (np.float32(1.01) * torch.sqrt((M * M).sum()) + np.float32(1e-6))).bfloat16()
        for a, b, c in O.COEFFICIENTS:
            A = (X.float() @ X.float().T.contiguous()).bfloat16()
            B = (np.float32(b) * A.float() + np.float32(c) * (A.float() @ A.float()).bfloat16().float()).bfloat16()
            Y = (B.float() @ X.float()).bfloat16()
            X = (np.float32(a) * X.float() + Y.float()).bfloat16()
        out.append((X.T if transposed else X).T.float())
    return torch.stack(out)


# sizes that are multiples of 128 run the library's own MFMA GEMM (128 x 64 tiles
# for grids below the CU count), the others rocBLAS
@pytest.mark.parametrize("m,n,k", [(64, 64, 3), (160, 48, 2), (128, 128, 3), (256, 384, 2), (384, 256, 2),
                                   (512, 512, 4), (512, 2048, 1), (2048, 512, 1),
                                   # training sizes: grids of 128 x 128 tiles at and above the CU count
                                   (512, 512, 16), (512, 512, 32), (2048, 512, 8)])
def test_polar_express_bf16_compute(gpu, m, n, k):
    g = torch.Generator().manual_seed(m * 5 + n)
    G = torch.randn(k, n, m, generator=g)
    out = polar_express(G.to(gpu), compute_type=torch.bfloat16).cpu()
    julia = G.numpy().transpose(0, 2, 1)
    ref = O.polar_express(julia).transpose(0, 2, 1)
    e64 = rel_err(out.numpy(), ref)
    eb = rel_err(out.numpy(), _torch_polar_bf16(G.to(gpu)).cpu().numpy())
    e_ref_bf16 = rel_err(_torch_polar_bf16(G.to(gpu)).cpu().numpy(), ref)
    say(f"polar bf16 {m}x{n}x{k}: vs float64 {e64:.2e}, vs torch bf16 {eb:.2e} (torch bf16 vs float64 {e_ref_bf16:.2e})")
    assert e64 < POLAR_TOL_BF16 and e64 <= 1.5 * e_ref_bf16 and eb < 1.5 * POLAR_TOL_BF16


def _torch_polar_bf16_steps(G, steps):
    out = []
    for g in G:
        M = g.T
        transposed = M.shape[0] > M.shape[1]
        X = ((M.T if transposed else M) / (np.float32(1.01) * torch.sqrt((M * M).sum()) + np.float32(1e-6))).bfloat16()
        for t in range(steps):
            a, b, c = O.COEFFICIENTS[min(t, len(O.COEFFICIENTS) - 1)]
            A = (X.float() @ X.float().T.contiguous()).bfloat16()
            B = (np.float32(b) * A.float() + np.float32(c) * (A.float() @ A.float()).bfloat16().float()).bfloat16()
            X = (np.float32(a) * X.float() + (B.float() @ X.float()).bfloat16().float()).bfloat16()
        out.append((X.T if transposed else X).T.float())
    return torch.stack(out)


@pytest.mark.parametrize("steps", [0, 1, 2, 7])
@pytest.mark.parametrize("m,n", [(256, 384), (384, 256)])
def test_polar_express_bf16_step_counts(gpu, m, n, steps):
    # the library's GEMM path writes G from the last step's product (as G or
    # its transpose); with no steps G is the normalised input rounded to bf16
    g = torch.Generator().manual_seed(steps * 31 + m)
    G = torch.randn(2, n, m, generator=g)
    out = polar_express(G.to(gpu), steps, compute_type=torch.bfloat16).cpu()
    julia = G.numpy().transpose(0, 2, 1)
    ref = O.polar_express(julia, steps).transpose(0, 2, 1)
    emu = _torch_polar_bf16_steps(G.to(gpu), steps).cpu().numpy()
    e64, eb = rel_err(out.numpy(), ref), rel_err(out.numpy(), emu)
    say(f"polar bf16 {m}x{n} steps={steps}: vs float64 {e64:.2e}, vs torch bf16 {eb:.2e}")
    if steps == 0:  # the normalised input, rounded once to bf16 (within one bf16 unit of float64)
        assert np.all(np.abs(out.numpy() - ref) <= 2.0 ** -8 * np.abs(ref))
    else:
        assert e64 < POLAR_TOL_BF16 and eb < 1.5 * POLAR_TOL_BF16


def test_grouped_bf16_many_stacks_equals_separate_calls(gpu):
    # six stacks on the library's GEMM, more than there are helper streams:
    # stacks that share a stream run in turn, the others concurrently
    g = torch.Generator().manual_seed(23)
    shapes = [(128, 128, 3), (256, 128, 2), (128, 384, 1), (256, 256, 2), (128, 512, 2), (384, 128, 1)]
    stacks = [torch.randn(k, n, m, generator=g).to(gpu) for m, n, k in shapes]
    separate = [polar_express(G, compute_type=torch.bfloat16) for G in stacks]
    grouped = [G.clone() for G in stacks]
    polar_express_grouped_(grouped, compute_type=torch.bfloat16)
    torch.cuda.synchronize()
    for a, b in zip(separate, grouped):
        assert torch.equal(a, b)


@pytest.mark.parametrize("compute_type", [torch.float32, torch.bfloat16])
def test_grouped_equals_separate_calls(gpu, compute_type):
    # the stacks run concurrently on helper streams, each with the same GEMMs as
    # a call of its own: the results are identical
    g = torch.Generator().manual_seed(17)
    # six stacks on four helpers; the last two run the library's own GEMM in bf16
    shapes = [(64, 64, 5), (48, 160, 3), (160, 48, 2), (96, 96, 1), (128, 256, 2), (384, 128, 3)]
    stacks = [torch.randn(k, n, m, generator=g).to(gpu) for m, n, k in shapes]
    separate = [polar_express(G, compute_type=compute_type) for G in stacks]
    grouped = [G.clone() for G in stacks]
    polar_express_grouped_(grouped, compute_type=compute_type)
    torch.cuda.synchronize()
    for a, b in zip(separate, grouped):
        assert torch.equal(a, b)
