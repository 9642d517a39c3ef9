"""GPU parity of the allocating API and the autograd wrapper.

The reference's user-facing entry is ``attention(Q, K, V, window)``
(src/kernels.jl:417), which goes through ``attention_state``
(src/kernels.jl:425-433): the default instruction for the array type and head
dim (ext/FemtoChatCUDAExt.jl:225-226), ``attention_inputs`` (float32 inputs
converted to the 16-bit format of the matrix-core path, :229-230), an O of the
input format or Float32 (:1238-1240) and float32 statistics
(``accumulator_type``, :228).  Its AD consumer is the Enzyme rule
(ext/FemtoChatEnzymeExt.jl:221-278), whose reverse pass runs ``Δattention!``
into zeroed gradient buffers.  Here those are ``kernels.attention``,
``attention_state`` and ``AttentionFunction``; every case is compared with the
float64 oracle on the values the kernels actually consume (bf16-rounded
inputs in fast mode) at the contract's tolerances.
"""
import numpy as np
import pytest
import torch

from femtochat_amd import MFMAExact, MFMAFast
from femtochat_amd import kernels as Kn
from femtochat_amd import workloads as W
from oracle import attention_ref as R
from tests.helpers import TOL, TOL_LSE, lse_err, rel_err, say, to_np

pytestmark = pytest.mark.gpu


def _inputs(seed, B, T, H, Hkv, D):
    rng = np.random.Generator(np.random.PCG64(seed))
    Q = rng.standard_normal((B, T, H, D), dtype=np.float32)
    K = rng.standard_normal((B, T, Hkv, D), dtype=np.float32)
    V = rng.standard_normal((B, T, Hkv, D), dtype=np.float32)
    dO = (0.1 * rng.standard_normal((B, T, H, D))).astype(np.float32)
    Q = Q / np.sqrt((Q.astype(np.float64) ** 2).mean(-1, keepdims=True)).astype(np.float32)
    K = K / np.sqrt((K.astype(np.float64) ** 2).mean(-1, keepdims=True)).astype(np.float32)
    return Q, K, V, dO


def _bf16_round(x):
    return torch.from_numpy(x).bfloat16().float().numpy()


SHAPES = [
    # B, T, H, Hkv, D, window, with positions
    (2, 200, 4, 2, 128, (-1, 0), False),
    (1, 333, 6, 3, 64, (100, 0), False),
    (2, 300, 4, 2, 128, (-1, 0), True),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "-".join(map(str, s)))
def test_attention_fp32_inputs_default_fast(gpu, shape):
    """attention(Q, K, V, window) with float32 GPU inputs: MFMAFast by default,
    inputs rounded to bf16 by the library, O returned in float32."""
    B, T, H, Hkv, D, window, with_pos = shape
    say(f"attention() fp32 default B={B} T={T} H={H} Hkv={Hkv} D={D} window={window} pos={with_pos}")
    Q, K, V, _ = _inputs(T + D, B, T, H, Hkv, D)
    pos = W.document_positions(T, B, seed=T, mean=50, sigma=1.0, cap=200) if with_pos else None
    Qd, Kd, Vd = (torch.from_numpy(x).to(gpu) for x in (Q, K, V))
    pos_d = None if pos is None else torch.from_numpy(pos).to(gpu)
    assert isinstance(Kn.instruction(Qd.dtype, gpu, D), MFMAFast)
    O = Kn.attention(Qd, Kd, Vd, window, positions=pos_d)
    torch.cuda.synchronize()
    assert O.dtype == torch.float32 and tuple(O.shape) == (B, T, H, D)
    O_ref, _, _ = R.forward(_bf16_round(Q), _bf16_round(K), _bf16_round(V), window, pos)
    e = rel_err(to_np(O), O_ref)
    assert e <= TOL["fast"], f"O rel err {e}"
    # The same run through the explicit pieces (library conversion, attention_)
    # is bit-identical: the allocating path adds nothing of its own.
    st = Kn.attention_state(MFMAFast(), Qd, Kd, Vd, window, positions=pos_d)
    Qb, Kb, Vb = (torch.empty(x.shape, dtype=torch.bfloat16, device=gpu) for x in (Qd, Kd, Vd))
    for dst, src in zip((Qb, Kb, Vb), (Qd, Kd, Vd)):
        Kn.convert_(dst, src)
    O2 = torch.empty(Q.shape, dtype=torch.float32, device=gpu)
    l2 = torch.empty((B, H, T), dtype=torch.float32, device=gpu)
    m2 = torch.empty((B, H, T), dtype=torch.float32, device=gpu)
    Kn.attention_(MFMAFast(), O2, l2, m2, Qb, Kb, Vb, window, positions=pos_d)
    torch.cuda.synchronize()
    assert st.Q.dtype == torch.bfloat16 and torch.equal(st.Q, Qb)
    assert torch.equal(O, O2) and torch.equal(st.O, O2)
    assert torch.equal(st.l, l2) and torch.equal(st.m, m2)


@pytest.mark.parametrize("shape", SHAPES[:2], ids=lambda s: "-".join(map(str, s)))
def test_attention_state_exact(gpu, shape):
    """attention_state(MFMAExact(), ...): float32 kept as is, O/l/m float32,
    O within 1e-4 and the log-sum-exp within 1e-5 of the oracle."""
    B, T, H, Hkv, D, window, _ = shape
    say(f"attention_state exact B={B} T={T} H={H} Hkv={Hkv} D={D} window={window}")
    Q, K, V, _ = _inputs(T + 7 * D, B, T, H, Hkv, D)
    Qd, Kd, Vd = (torch.from_numpy(x).to(gpu) for x in (Q, K, V))
    st = Kn.attention_state(MFMAExact(), Qd, Kd, Vd, window)
    torch.cuda.synchronize()
    assert isinstance(st.A, MFMAExact) and st.Q is Qd and st.K is Kd and st.V is Vd
    assert st.O.dtype == torch.float32 and st.l.dtype == torch.float32 and tuple(st.l.shape) == (B, H, T)
    O_ref, l_ref, m_ref = R.forward(Q, K, V, window)
    assert rel_err(to_np(st.O), O_ref) <= TOL["exact"]
    assert lse_err(to_np(st.l), to_np(st.m), l_ref, m_ref) <= TOL_LSE
    # attention(A, ...) returns the same O
    O = Kn.attention(MFMAExact(), Qd, Kd, Vd, window)
    torch.cuda.synchronize()
    assert torch.equal(O, st.O)


@pytest.mark.parametrize("mode,in_dtype", [("fast", torch.float32), ("fast", torch.bfloat16), ("exact", torch.float32)])
@pytest.mark.parametrize("with_pos", [False, True])
def test_autograd_wrapper(gpu, mode, in_dtype, with_pos):
    """AttentionFunction: forward = attention_state, backward = delta_attention_
    into zeroed float32 buffers, gradients cast back to the inputs' dtypes;
    end to end against the oracle's forward and backward."""
    B, T, H, Hkv, D, window = 2, 260, 4, 2, 128, (-1, 0)
    say(f"autograd mode={mode} dtype={in_dtype} pos={with_pos}")
    Q, K, V, dO = _inputs(11 + int(with_pos), B, T, H, Hkv, D)
    pos = W.document_positions(T, B, seed=5, mean=60, sigma=1.0, cap=200) if with_pos else None
    A = MFMAFast() if mode == "fast" else MFMAExact()
    leaves = [torch.from_numpy(x).to(gpu).to(in_dtype).requires_grad_(True) for x in (Q, K, V)]
    pos_d = None if pos is None else torch.from_numpy(pos).to(gpu)
    O = Kn.AttentionFunction.apply(*leaves, window, A, pos_d)
    dOd = torch.from_numpy(dO).to(gpu).to(O.dtype)
    O.backward(dOd)
    torch.cuda.synchronize()
    for x in leaves:
        assert x.grad is not None and x.grad.dtype == in_dtype and x.grad.shape == x.shape
    if mode == "fast":
        # dO reaches the kernels in bf16 either way: a bf16 O takes a bf16 dO,
        # and an fp32 dO is rounded to bf16 by the library.
        Qr, Kr, Vr, dOr = (_bf16_round(x) for x in (Q, K, V, dO))
    else:
        Qr, Kr, Vr, dOr = Q, K, V, dO
    O_ref, l_ref, m_ref = R.forward(Qr, Kr, Vr, window, pos)
    tol = TOL[mode]
    assert rel_err(to_np(O), O_ref) <= tol
    g_ref = R.backward(dOr, Qr, Kr, Vr, O_ref, l_ref, m_ref, window, pos)
    for name, x, r in zip(("dQ", "dK", "dV"), leaves, g_ref):
        e = rel_err(to_np(x.grad), r)
        assert e <= tol, f"{name} rel err {e}"


def test_autograd_matches_explicit_backward(gpu):
    """The wrapper's gradients equal an explicit delta_attention_ into zeroed
    float32 buffers on the saved state, bit for bit."""
    B, T, H, Hkv, D, window = 1, 200, 4, 2, 64, (64, 0)
    Q, K, V, dO = _inputs(3, B, T, H, Hkv, D)
    leaves = [torch.from_numpy(x).to(gpu).requires_grad_(True) for x in (Q, K, V)]
    O = Kn.AttentionFunction.apply(*leaves, window, MFMAFast(), None)
    dOd = torch.from_numpy(dO).to(gpu)
    O.backward(dOd)
    st = Kn.attention_state(MFMAFast(), *(x.detach() for x in leaves), window)
    grads = [torch.zeros(x.shape, dtype=torch.float32, device=gpu) for x in (st.Q, st.K, st.V)]
    Kn.delta_attention_(MFMAFast(), *grads, dOd, st.Q, st.K, st.V, st.O, st.l, st.m, window)
    torch.cuda.synchronize()
    assert torch.equal(O.detach(), st.O)
    for x, g in zip(leaves, grads):
        assert torch.equal(x.grad, g)


def test_attention_fp16_inputs(gpu):
    """float16 inputs select the matrix-core path as in the reference
    (ext/FemtoChatCUDAExt.jl:214-223); this library's matrix-core format is
    bf16, so they are converted to it (one rounding of each value, which the
    oracle reproduces) and O comes back in float32."""
    B, T, H, Hkv, D, window = 2, 150, 4, 2, 64, (-1, 0)
    Q, K, V, _ = _inputs(16, B, T, H, Hkv, D)
    Qh, Kh, Vh = (torch.from_numpy(x).half() for x in (Q, K, V))
    assert isinstance(Kn.instruction(torch.float16, gpu, D), MFMAFast)
    O = Kn.attention(Qh.to(gpu), Kh.to(gpu), Vh.to(gpu), window)
    torch.cuda.synchronize()
    assert O.dtype == torch.float32 and tuple(O.shape) == (B, T, H, D)
    r = [x.float().bfloat16().float().numpy() for x in (Qh, Kh, Vh)]
    O_ref, _, _ = R.forward(r[0], r[1], r[2], window)
    e = rel_err(to_np(O), O_ref)
    assert e <= TOL["fast"], f"O rel err {e}"
