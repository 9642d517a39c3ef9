"""Work order of the fast kernels with positions (packed documents).

With positions, fast mode takes the tiles of all batch rows longest first:
the forward and dQ query tiles (128 queries) by the number of 64-key tiles
they visit, the dK/dV key tiles (128 keys) by the number of 128-query tiles
that can see them.  The order only changes which workgroup runs a tile when,
never what a tile computes, so:
  * the forward's outputs are bit-identical with the order (a workspace) and
    without it (no workspace, the default order);
  * the ordered forward and backward match the oracle;
  * the order tables the library leaves in the workspace are permutations of
    the tiles, sorted by the work the kernels actually do.  The work is
    recounted here from the visibility mask itself (which keys each query
    sees), not from the library's bound tables.
"""
import ctypes

import numpy as np
import pytest
import torch

import femtochat_amd._lib as L
from femtochat_amd import MFMAFast
from femtochat_amd import kernels as Kn
from femtochat_amd import workloads as W
from oracle import attention_ref as R
from tests.helpers import TOL, TOL_LSE, gpu_backward, lse_err, rel_err, say, to_np

pytestmark = pytest.mark.gpu

CASES = [
    # B, T, H, Hkv, D, window, mean document length
    (3, 1000, 4, 2, 128, (-1, 0), 90),
    (2, 777, 2, 1, 64, (300, 0), 150),
    (1, 515, 2, 2, 32, (200, 40), 60),
    (4, 256, 2, 1, 128, (-1, 0), 500),
    (1, 1, 2, 1, 64, (-1, 0), 5),        # one query
    (2, 129, 2, 2, 16, (-1, 0), 10),     # one query past a tile
    (3, 300, 4, 1, 32, (0, 0), 30),      # each query sees only itself
]


def _align(x):
    return (x + 255) // 256 * 256


def _first_visible(T, window, pos_row):
    """Per query: its smallest visible key as the kernels bound it (the
    document start, the window's left edge, 0), or T past the end; and its
    largest visible key."""
    left, right = window
    if left == -1 and right == 0:
        left = T
    q = np.arange(T)
    lb = np.maximum(np.maximum(q - left, q - pos_row.astype(np.int64)), 0)
    ub = np.minimum(q + right, T - 1)
    return lb, ub


def _expected_orders(T, window, positions):
    """(qorder, korder) recounted from each query's visible range."""
    left, right = window
    if left == -1 and right == 0:
        left = T
    B = positions.shape[0]
    n128 = -(-T // 128)
    qwork, kwork = [], []
    for b in range(B):
        lb, ub = _first_visible(T, window, positions[b])
        lb_pad = np.full(n128 * 128, T)
        lb_pad[:T] = lb
        for t in range(n128):
            rows = slice(128 * t, min(128 * t + 128, T))
            kmin, kmax = int(lb[rows].min()), int(ub[rows].max())
            # 64-key tiles from the one holding the first key to the one holding the last.
            qwork.append(kmax // 64 - kmin // 64 + 1 if kmax >= kmin else 0)
        for t in range(n128):
            k0, k1 = 128 * t, min(128 * t + 128, T) - 1
            qlo, qhi = max(0, k0 - right), min(T - 1, k1 + left)
            n = 0
            for u in range(qlo // 128, qhi // 128 + 1) if qhi >= qlo else ():
                n += int(lb_pad[128 * u:128 * u + 128].min() <= k1)
            kwork.append(n)
    qwork, kwork = np.array(qwork), np.array(kwork)
    return np.argsort(-qwork, kind="stable"), np.argsort(-kwork, kind="stable"), qwork, kwork


def _inputs(seed, B, T, H, Hkv, D):
    rng = np.random.Generator(np.random.PCG64(seed))
    Q = rng.standard_normal((B, T, H, D), dtype=np.float32)
    K = rng.standard_normal((B, T, Hkv, D), dtype=np.float32)
    V = rng.standard_normal((B, T, Hkv, D), dtype=np.float32)
    dO = (rng.standard_normal((B, T, H, D), dtype=np.float32) * 0.1).astype(np.float32)
    Q = Q / np.sqrt((Q.astype(np.float64) ** 2).mean(-1, keepdims=True)).astype(np.float32)
    K = K / np.sqrt((K.astype(np.float64) ** 2).mean(-1, keepdims=True)).astype(np.float32)
    return tuple(torch.from_numpy(x).bfloat16().float().numpy() for x in (Q, K, V, dO))


def _forward_abi(A, Q, K, V, window, pos, workspace):
    """fc_attn_fwd through the C ABI, with the given workspace tensor or none."""
    B, T, H, D = Q.shape
    O = torch.full(Q.shape, float("nan"), dtype=torch.bfloat16, device=Q.device)
    l = torch.full((B, H, T), float("nan"), device=Q.device)
    m = torch.full((B, H, T), float("nan"), device=Q.device)
    d = Kn._desc(A, Q, K, window, L.FC_BF16, L.FC_BF16, L.FC_BF16)
    ws, nbytes = None, 0
    if workspace is not None:
        ws = ctypes.c_void_p(workspace.data_ptr())
        nbytes = workspace.numel()
    L.check(L.lib().fc_attn_fwd(ctypes.byref(d), Kn._ptr(Q), Kn._ptr(K), Kn._ptr(V), Kn._ptr(pos), Kn._ptr(O),
                                Kn._ptr(l), Kn._ptr(m), ws, ctypes.c_size_t(nbytes),
                                Kn._stream_ptr(Q.device)))
    return O, l, m


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c)))
def test_work_order(gpu, case):
    B, T, H, Hkv, D, window, mean = case
    say(f"order case B={B} T={T} H={H} Hkv={Hkv} D={D} window={window} mean={mean}")
    A = MFMAFast()
    positions = W.document_positions(T, B, seed=T + B, mean=mean, sigma=1.0, cap=4 * mean)
    Q, K, V, dO = _inputs(T, B, T, H, Hkv, D)
    Qd, Kd, Vd, dOd = (torch.from_numpy(x).to(gpu, torch.bfloat16).contiguous() for x in (Q, K, V, dO))
    pos_d = torch.from_numpy(positions).to(gpu).contiguous()
    n128 = -(-T // 128)
    q_exp, k_exp, qwork, kwork = _expected_orders(T, window, positions)

    # Forward: the same outputs with the order and without it.
    nbytes = Kn.forward_workspace_bytes(A, Qd, Kd, positions=pos_d) - 256
    chunk_bytes = B * (-(-T // 32)) * 2 * 4
    assert nbytes == _align(chunk_bytes) + _align(B * n128 * 4)
    fws = torch.empty(nbytes, dtype=torch.uint8, device=gpu)  # torch allocations are 256-byte aligned
    assert fws.data_ptr() % 256 == 0
    O1, l1, m1 = _forward_abi(A, Qd, Kd, Vd, window, pos_d, fws)
    O0, l0, m0 = _forward_abi(A, Qd, Kd, Vd, window, pos_d, None)
    torch.cuda.synchronize()
    assert torch.equal(O1, O0) and torch.equal(l1, l0) and torch.equal(m1, m0), "order changed the forward's results"
    qorder = fws[_align(chunk_bytes):_align(chunk_bytes) + B * n128 * 4].view(torch.int32).cpu().numpy()
    assert sorted(qorder.tolist()) == list(range(B * n128)), "forward order is not a permutation"
    assert np.all(np.diff(qwork[qorder]) <= 0), "forward order is not longest first"
    assert np.array_equal(qorder, q_exp)

    # And both match the oracle.
    O_ref, l_ref, m_ref = R.forward(Q, K, V, window, positions)
    assert rel_err(to_np(O1), O_ref) <= TOL["fast"]
    assert lse_err(to_np(l1), to_np(m1), l_ref, m_ref) <= TOL_LSE

    # Backward: the orders it leaves in its workspace, and its gradients.
    need = Kn.backward_workspace_bytes(A, Qd, Kd, positions=pos_d)
    bws = torch.empty(need, dtype=torch.uint8, device=gpu)
    dQ = torch.zeros_like(Qd)
    dK = torch.zeros_like(Kd)
    dV = torch.zeros_like(Vd)
    Kn.delta_attention_(A, dQ, dK, dV, dOd, Qd, Kd, Vd, O1, l1, m1, window, positions=pos_d, accumulate=False,
                        workspace=bws)
    torch.cuda.synchronize()
    base = (bws.data_ptr() + 255) // 256 * 256 - bws.data_ptr()
    nq = B * H * T
    off = base + 2 * _align(nq * 4) + _align(chunk_bytes) + _align(8 * 4)  # Delta, lse2, bounds, counters
    bq = bws[off:off + B * n128 * 4].view(torch.int32).cpu().numpy()
    off += _align(B * n128 * 4)
    bk = bws[off:off + B * n128 * 4].view(torch.int32).cpu().numpy()
    assert np.array_equal(bq, q_exp)
    assert sorted(bk.tolist()) == list(range(B * n128)), "dK/dV order is not a permutation"
    assert np.all(np.diff(kwork[bk]) <= 0), "dK/dV order is not longest first"
    assert np.array_equal(bk, k_exp)
    g_ref = R.backward(dO, Q, K, V, to_np(O1), to_np(l1), to_np(m1), window, positions)
    for name, x, r in zip(("dQ", "dK", "dV"), (dQ, dK, dV), g_ref):
        e = rel_err(to_np(x), r)
        assert e <= TOL["fast"], f"{name} rel err {e}"


def test_order_repeats_and_shrinks(gpu):
    """Two ordered calls in a row, the second on a smaller problem, give the
    same gradients as fresh calls (the order tables are rewritten per call)."""
    A = MFMAFast()
    outs = []
    for (B, T) in ((3, 900), (2, 300), (3, 900)):
        positions = W.document_positions(T, B, seed=5, mean=80, sigma=1.0, cap=400)
        Q, K, V, dO = _inputs(7, B, T, 2, 1, 64)
        Qd, Kd, Vd, dOd = (torch.from_numpy(x).to(gpu, torch.bfloat16).contiguous() for x in (Q, K, V, dO))
        pos_d = torch.from_numpy(positions).to(gpu)
        O, l, m = _forward_abi(A, Qd, Kd, Vd, (-1, 0), pos_d,
                               torch.empty(Kn.forward_workspace_bytes(A, Qd, Kd, positions=pos_d) - 256,
                                           dtype=torch.uint8, device=gpu))
        g = gpu_backward(A, dOd, Qd, Kd, Vd, O, l, m, (-1, 0), pos_d)
        torch.cuda.synchronize()
        outs.append((O, l, m) + tuple(g))
    for a, b in zip(outs[0], outs[2]):
        assert torch.equal(a, b)


def test_order_limit_gives_the_same_bits(gpu):
    """Past the order kernel's table (B * ceil(T/128) > 4096) the kernels fall
    back to the index order; per-row results must not depend on which: the
    33-row problem (unordered) equals its two halves run separately (each
    ordered), bit for bit."""
    A = MFMAFast()
    B, T, H, Hkv, D = 33, 16384, 1, 1, 16
    assert B * (-(-T // 128)) > 4096 and 17 * (-(-T // 128)) <= 4096
    positions = W.document_positions(T, B, seed=11, mean=600, sigma=1.0, cap=6000)
    g = torch.Generator(device=gpu).manual_seed(3)
    Qd, Kd, Vd = (torch.randn(B, T, n, D, device=gpu, generator=g).bfloat16() for n in (H, Hkv, Hkv))
    dOd = (0.1 * torch.randn(B, T, H, D, device=gpu, generator=g)).bfloat16()
    pos_d = torch.from_numpy(positions).to(gpu)
    assert Kn.forward_workspace_bytes(A, Qd, Kd, positions=pos_d) == 0
    fwd = _forward_abi(A, Qd, Kd, Vd, (-1, 0), pos_d, None)
    full = fwd + gpu_backward(A, dOd, Qd, Kd, Vd, *fwd, (-1, 0), pos_d)
    for rows in (slice(0, 16), slice(16, 33)):
        sub = [x[rows].contiguous() for x in (Qd, Kd, Vd, dOd, pos_d)]
        ws = torch.empty(Kn.forward_workspace_bytes(A, sub[0], sub[1], positions=sub[4]) - 256, dtype=torch.uint8,
                         device=gpu)
        O, l, m = _forward_abi(A, sub[0], sub[1], sub[2], (-1, 0), sub[4], ws)
        part = (O, l, m) + gpu_backward(A, sub[3], sub[0], sub[1], sub[2], O, l, m, (-1, 0), sub[4])
        torch.cuda.synchronize()
        for name, a, b in zip(("O", "l", "m", "dQ", "dK", "dV"), part, full):
            assert torch.equal(a, b[rows]), f"the order changed {name}"


@pytest.mark.parametrize("window,T,B", [((100, 0), 700, 3), ((300, 20), 1024, 3), ((200, 0), 1024, 4), ((0, 3), 640, 8)])
def test_row_local_order_gives_the_same_bits(gpu, window, T, B):
    """A window of at most half the sequence takes the row-local order (the
    forward, with B*Hkv divisible by 8 its full query tiles first and then the
    partial ones, and dK/dV); positions that restart nowhere (positions[q] = q) leave the
    mask unchanged but take the work order instead.  Same mask, same bits."""
    A = MFMAFast()
    H, Hkv, D = 4, 2, 64
    assert window[0] + max(window[1], 0) + 1 <= T // 2  # the row-local order applies
    Q, K, V, dO = _inputs(T + 7, B, T, H, Hkv, D)
    Qd, Kd, Vd, dOd = (torch.from_numpy(x).to(gpu, torch.bfloat16).contiguous() for x in (Q, K, V, dO))
    linear = torch.arange(T, dtype=torch.int32, device=gpu).repeat(B, 1).contiguous()
    outs = []
    for pos in (None, linear):
        ws = None
        n = Kn.forward_workspace_bytes(A, Qd, Kd, positions=pos)
        if n:
            ws = torch.empty(n - 256, dtype=torch.uint8, device=gpu)
        fwd = _forward_abi(A, Qd, Kd, Vd, window, pos, ws)
        outs.append(fwd + gpu_backward(A, dOd, Qd, Kd, Vd, *fwd, window, pos))
    torch.cuda.synchronize()
    for name, a, b in zip(("O", "l", "m", "dQ", "dK", "dV"), *outs):
        assert torch.equal(a, b), f"{name} differs between the row-local and the work order"
    O_ref, l_ref, m_ref = R.forward(Q, K, V, window, None)
    assert rel_err(to_np(outs[0][0]), O_ref) <= TOL["fast"]
