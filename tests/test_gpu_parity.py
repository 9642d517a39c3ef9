"""GPU parity: the HIP kernels (through the C ABI) against the float64 oracle.

Small cases cover every code path (head dims, GQA ratios, ragged T, windows
including empty rows, document masks, both modes, bf16/fp32 storage); the
committed golden fixtures are reproduced; the full-size BASELINE workloads
C1..C5 are checked against the oracle on (batch, KV group) slices in every
residue class of the kernels' grid rows mod 8 (the XCD a row runs on) plus a
middle batch row, and over the whole output through size-independent
properties: the sum identities of dV and dK, the scale identity
<dQ, Q> = <dK, K> per (batch, KV group), and the closed form of every row
whose query sees a single key (the first query of a row, every document
start): O = V, l = 1, m = tau q.k, dQ = 0.
"""
import zlib
from pathlib import Path

import numpy as np
import pytest
import torch

from femtochat_amd import MFMAExact, MFMAFast
from femtochat_amd import workloads as W
from oracle import attention_ref as R
from tests.helpers import TOL, TOL_LSE, gpu_backward, gpu_forward, lse_err, rel_err, say, to_np

pytestmark = pytest.mark.gpu


def _inputs(seed, B, T, H, Hkv, D, fast, rms=True, dO_std=0.1):
    rng = np.random.Generator(np.random.PCG64(seed))
    Q = rng.standard_normal((B, T, H, D), dtype=np.float32)
    K = rng.standard_normal((B, T, Hkv, D), dtype=np.float32)
    V = rng.standard_normal((B, T, Hkv, D), dtype=np.float32)
    dO = (rng.standard_normal((B, T, H, D), dtype=np.float32) * dO_std).astype(np.float32)
    if rms:
        Q = Q / np.sqrt((Q.astype(np.float64) ** 2).mean(-1, keepdims=True)).astype(np.float32)
        K = K / np.sqrt((K.astype(np.float64) ** 2).mean(-1, keepdims=True)).astype(np.float32)
    if fast:
        Q, K, V, dO = (torch.from_numpy(x).bfloat16().float().numpy() for x in (Q, K, V, dO))
    return Q, K, V, dO


def _dev(x, fast, device):
    return torch.from_numpy(x).to(device=device, dtype=torch.bfloat16 if fast else torch.float32).contiguous()


def _check_case(device, mode, B, T, H, Hkv, D, window, positions=None, seed=0, out_dtype=None, grad_dtype=None,
                dout_dtype=None):
    fast = mode == "fast"
    A = MFMAFast() if fast else MFMAExact()
    say(f"case mode={mode} B={B} T={T} H={H} Hkv={Hkv} D={D} window={window} pos={positions is not None} "
        f"out={out_dtype} grad={grad_dtype} dO={dout_dtype}")
    Q, K, V, dO = _inputs(seed, B, T, H, Hkv, D, fast)
    Qd, Kd, Vd = (_dev(x, fast, device) for x in (Q, K, V))
    pos_d = None if positions is None else torch.from_numpy(positions).to(device).contiguous()
    O, l, m = gpu_forward(A, Qd, Kd, Vd, window, pos_d, out_dtype=out_dtype)
    torch.cuda.synchronize()
    O_ref, l_ref, m_ref = R.forward(Q, K, V, window, positions)
    tol = TOL[mode]
    eO = rel_err(to_np(O), O_ref)
    eL = lse_err(to_np(l), to_np(m), l_ref, m_ref)
    empty = l_ref == 0
    assert eO <= tol, f"O rel err {eO}"
    assert eL <= TOL_LSE, f"LSE err {eL}"
    assert np.all(to_np(l)[empty] == 0) and np.all(to_np(m)[empty] == -R.FLT_MAX), "empty rows must give l=0, m=-floatmax"
    assert np.all(to_np(O)[np.transpose(empty, (0, 2, 1))] == 0), "empty rows must give O=0"

    # Backward with the GPU's own saved state on both sides.
    dOd = torch.from_numpy(dO).to(device=device, dtype=(dout_dtype or (torch.bfloat16 if fast else torch.float32)))
    dQ, dK, dV = gpu_backward(A, dOd, Qd, Kd, Vd, O, l, m, window, pos_d, grad_dtype=grad_dtype)
    torch.cuda.synchronize()
    # Fast mode against the restatement of the reference's tensor-core
    # backward (P and dS rounded to bf16, dS = 0 on rows with one visible key):
    # where every row sees a single key, dQ and dK are exactly zero there and
    # the unrounded float64 gradients are rounding noise (about 1e-8 with fp32
    # O, whose 1/l is not exactly 1), which the relative metric would inflate.
    g_ref = R.backward(dO, Q, K, V, to_np(O), to_np(l), to_np(m), window, positions, fast=fast)
    for name, x, r in zip(("dQ", "dK", "dV"), (dQ, dK, dV), g_ref):
        e = rel_err(to_np(x), r)
        assert e <= tol, f"{name} rel err {e}"


SMALL_CASES = [
    # mode, B, T, H, Hkv, D, window
    ("exact", 2, 4, 2, 1, 16, (4, 0)),
    ("exact", 1, 1, 1, 1, 16, (-1, 0)),
    ("exact", 2, 130, 4, 2, 32, (-1, 0)),
    ("exact", 1, 257, 2, 2, 64, (40, 0)),
    ("exact", 2, 200, 4, 1, 128, (-1, 0)),
    ("exact", 1, 96, 2, 2, 128, (16, 7)),
    ("exact", 1, 70, 2, 1, 64, (0, 0)),
    ("exact", 1, 50, 2, 2, 32, (-1, 5)),
    ("fast", 2, 4, 2, 1, 16, (4, 0)),
    ("fast", 1, 1, 2, 1, 128, (-1, 0)),
    ("fast", 2, 130, 4, 2, 32, (-1, 0)),
    ("fast", 1, 257, 6, 2, 64, (40, 0)),
    ("fast", 2, 300, 4, 1, 128, (-1, 0)),
    ("fast", 1, 192, 2, 2, 128, (64, 0)),
    ("fast", 1, 96, 2, 2, 128, (16, 7)),
    ("fast", 1, 70, 2, 1, 64, (0, 0)),
    ("fast", 1, 50, 2, 2, 32, (-1, 5)),
    ("fast", 1, 129, 3, 3, 128, (1000, 1000)),
]


@pytest.mark.parametrize("case", SMALL_CASES, ids=lambda c: "-".join(map(str, c)))
def test_small_cases(gpu, case):
    mode, B, T, H, Hkv, D, window = case
    _check_case(gpu, mode, B, T, H, Hkv, D, window, seed=zlib.crc32(repr(case).encode()) % 1000)


PADDED_CASES = [
    # mode, B, T, H, Hkv, D, window: head dims between the compiled widths
    ("exact", 2, 130, 4, 2, 48, (-1, 0)),
    ("exact", 1, 100, 2, 2, 80, (16, 7)),
    ("exact", 1, 200, 2, 1, 96, (40, 0)),
    ("exact", 1, 77, 3, 1, 112, (-1, 0)),
    ("fast", 2, 130, 4, 2, 48, (-1, 0)),
    ("fast", 1, 100, 2, 2, 80, (16, 7)),
    ("fast", 1, 200, 6, 2, 96, (40, 0)),
    ("fast", 1, 77, 3, 1, 112, (-1, 0)),
]


@pytest.mark.parametrize("case", PADDED_CASES, ids=lambda c: "-".join(map(str, c)))
def test_padded_head_dims(gpu, case):
    """D in {48, 80, 96, 112} (the reference's tensor-core path takes any
    D % 16 == 0 up to 128, ext/FemtoChatCUDAExt.jl:214-223): the library runs
    them zero-padded to 64 or 128 with the scale of the real D."""
    mode, B, T, H, Hkv, D, window = case
    _check_case(gpu, mode, B, T, H, Hkv, D, window, seed=zlib.crc32(repr(case).encode()) % 1000)


def test_padded_head_dims_storage_positions_accumulate(gpu):
    """The padded path with fp32 O/dO/gradients in fast mode, with a document
    mask, and adding into existing bf16 gradients (the padded kernels write
    float32 gradients that are added to the caller's values and rounded once)."""
    pos = W.document_positions(180, 2, seed=96, mean=40, sigma=1.0, cap=120)
    _check_case(gpu, "fast", 2, 180, 4, 2, 96, (-1, 0), positions=pos, out_dtype=torch.float32,
                grad_dtype=torch.float32, dout_dtype=torch.float32, seed=96)
    B, T, H, Hkv, D = 1, 150, 4, 2, 80
    A = MFMAFast()
    Q, K, V, dO = _inputs(9, B, T, H, Hkv, D, True)
    Qd, Kd, Vd, dOd = (_dev(x, True, gpu) for x in (Q, K, V, dO))
    O, l, m = gpu_forward(A, Qd, Kd, Vd, (-1, 0))
    base = [torch.randn(x.shape, device=gpu).to(x.dtype) for x in (Qd, Kd, Vd)]
    fresh = gpu_backward(A, dOd, Qd, Kd, Vd, O, l, m, (-1, 0), accumulate=False, init=base)
    added = gpu_backward(A, dOd, Qd, Kd, Vd, O, l, m, (-1, 0), accumulate=True, init=base)
    torch.cuda.synchronize()
    g_ref = R.backward(dO, Q, K, V, to_np(O), to_np(l), to_np(m), (-1, 0))
    for f, a, b0, r in zip(fresh, added, base, g_ref):
        assert rel_err(to_np(f), r) <= TOL["fast"]
        assert rel_err(to_np(a), to_np(f) + to_np(b0)) <= 1e-2


@pytest.mark.parametrize("window", [(-300, 400), (-255, 300), (-701, 700)])
def test_window_right_of_query_row_local_order(gpu, window):
    """Windows that start right of their query (left <= -255) in fast mode, with
    B*Hkv = 16 (a multiple of 8) and left + right + 1 <= T/2, so the forward
    and dK/dV take the row-local order: every query tile must be computed
    exactly once (the first full tile clamps to 0 for left < 0).  (-701, 700)
    at T = 700 leaves every row empty (left clamps to -T-1)."""
    _check_case(gpu, "fast", 4, 700, 4, 4, 64, window, seed=abs(window[0]))


@pytest.mark.parametrize("mode", ["exact", "fast"])
@pytest.mark.parametrize("T,D,window", [(300, 64, (-1, 0)), (517, 128, (100, 0)), (260, 128, (-1, 0))])
def test_document_mask(gpu, mode, T, D, window):
    pos = W.document_positions(T, 2, seed=T + D, mean=40, sigma=1.0, cap=200)
    _check_case(gpu, mode, 2, T, 4, 2, D, window, positions=pos, seed=T)


def test_fast_mode_storage_dtypes(gpu):
    # O, dO and gradients stored in fp32 while Q/K/V are bf16.
    _check_case(gpu, "fast", 1, 150, 4, 2, 128, (-1, 0), out_dtype=torch.float32, grad_dtype=torch.float32,
                dout_dtype=torch.float32)
    _check_case(gpu, "fast", 1, 150, 4, 2, 64, (-1, 0), out_dtype=torch.float32, grad_dtype=torch.bfloat16,
                dout_dtype=torch.bfloat16)


@pytest.mark.parametrize("mode,H,Hkv,D", [("fast", 32, 1, 64), ("fast", 16, 2, 128), ("exact", 24, 3, 32),
                                          ("fast", 12, 12, 16)])
def test_wide_gqa_groups(gpu, mode, H, Hkv, D):
    """GQA groups of 1 to 32 query heads per KV head: the dK/dV kernels sum the
    group's heads in registers (one item loops over all of them), and the
    forward and dQ map every query head to its KV head."""
    _check_case(gpu, mode, 2, 160, H, Hkv, D, (-1, 0), seed=H * 7 + Hkv)
    _check_case(gpu, mode, 1, 97, H, Hkv, D, (40, 3), seed=H * 7 + Hkv + 1)


@pytest.mark.parametrize("D", [16, 32, 64, 128])
def test_fp32_gradients_every_compiled_head_dim(gpu, D):
    """fp32 dQ, dK, dV at every compiled head dim.  The epilogues stage the
    accumulators through LDS, every lane writing its values and other lanes
    reading whole rows; at D = 16 the dV pass once reused, on the lanes that
    write nothing (d >= 16), the dK pass's read of the same LDS address, so
    rows 4-7 and 12-15 of every wave's keys came out as dK."""
    _check_case(gpu, "fast", 1, 150, 2, 1, D, (-1, 0), grad_dtype=torch.float32, seed=D)
    _check_case(gpu, "fast", 2, 96, 3, 3, D, (40, 0), out_dtype=torch.float32, grad_dtype=torch.float32,
                dout_dtype=torch.float32, seed=D + 1)


@pytest.mark.parametrize("D,docs", [(16, False), (64, True), (128, False), (128, True)])
def test_persistent_items_storage_and_accumulate(gpu, D, docs):
    """More dK/dV items than workgroups (5 batch rows x 8 KV heads x 8 key
    tiles = 320 items on 256 CUs), so a workgroup takes a second item while
    its first item's gradients leave through LDS; with documents the items
    come in the work order.  fp32 and bf16 gradients, overwritten and added
    to the buffers' values (the fp32 sum is the same addition the caller
    would do, so it must match bit for bit)."""
    B, T, H, Hkv = 5, 1024, 8, 8
    A = MFMAFast()
    Q, K, V, dO = _inputs(D + docs, B, T, H, Hkv, D, True)
    pos = W.document_positions(T, B, seed=D, mean=300, sigma=1.0, cap=T) if docs else None
    pos_d = None if pos is None else torch.from_numpy(pos).to(gpu).contiguous()
    Qd, Kd, Vd, dOd = (_dev(x, True, gpu) for x in (Q, K, V, dO))
    O, l, m = gpu_forward(A, Qd, Kd, Vd, (-1, 0), pos_d)
    torch.cuda.synchronize()
    g_ref = R.backward(dO, Q, K, V, to_np(O), to_np(l), to_np(m), (-1, 0), pos, fast=True)
    for gd in (torch.float32, torch.bfloat16):
        say(f"D={D} docs={docs} grads={gd}")
        base = [torch.randn(x.shape, device=gpu).to(gd) for x in (Qd, Kd, Vd)]
        fresh = gpu_backward(A, dOd, Qd, Kd, Vd, O, l, m, (-1, 0), pos_d, grad_dtype=gd)
        added = gpu_backward(A, dOd, Qd, Kd, Vd, O, l, m, (-1, 0), pos_d, grad_dtype=gd, accumulate=True, init=base)
        torch.cuda.synchronize()
        for name, f, s, b0, r in zip(("dQ", "dK", "dV"), fresh, added, base, g_ref):
            e = rel_err(to_np(f), r)
            assert e <= TOL["fast"], f"{name} rel err {e}"
            want = to_np(f) + to_np(b0)
            if gd == torch.float32:
                assert np.array_equal(to_np(s), want), f"{name}: accumulated fp32 differs from fresh + base"
            else:
                assert rel_err(to_np(s), want) <= 1e-2, f"{name}: accumulated bf16"


@pytest.mark.parametrize("mode", ["exact", "fast"])
def test_accumulate_and_overwrite(gpu, mode):
    fast = mode == "fast"
    A = MFMAFast() if fast else MFMAExact()
    B, T, H, Hkv, D = 1, 150, 4, 2, 64
    Q, K, V, dO = _inputs(7, B, T, H, Hkv, D, fast)
    Qd, Kd, Vd, dOd = (_dev(x, fast, gpu) for x in (Q, K, V, dO))
    O, l, m = gpu_forward(A, Qd, Kd, Vd, (-1, 0))
    base = [torch.randn(x.shape, device=gpu).to(x.dtype) for x in (Qd, Kd, Vd)]
    fresh = gpu_backward(A, dOd, Qd, Kd, Vd, O, l, m, (-1, 0), accumulate=False, init=base)
    added = gpu_backward(A, dOd, Qd, Kd, Vd, O, l, m, (-1, 0), accumulate=True, init=base)
    torch.cuda.synchronize()
    tol = 1e-6 if not fast else 1e-2
    for f, a, b0 in zip(fresh, added, base):
        e = rel_err(to_np(a), to_np(f) + to_np(b0))
        assert e <= tol, e


@pytest.mark.parametrize("mode", ["exact", "fast"])
def test_deterministic(gpu, mode):
    fast = mode == "fast"
    A = MFMAFast() if fast else MFMAExact()
    Q, K, V, dO = _inputs(11, 2, 333, 4, 2, 128, fast)
    Qd, Kd, Vd, dOd = (_dev(x, fast, gpu) for x in (Q, K, V, dO))
    r1 = gpu_forward(A, Qd, Kd, Vd, (-1, 0))
    r2 = gpu_forward(A, Qd, Kd, Vd, (-1, 0))
    g1 = gpu_backward(A, dOd, Qd, Kd, Vd, *r1, (-1, 0))
    g2 = gpu_backward(A, dOd, Qd, Kd, Vd, *r1, (-1, 0))
    torch.cuda.synchronize()
    for x, y in zip(r1 + g1, r2 + g2):
        assert torch.equal(x, y), "results must be bitwise reproducible"


WS_CASES = {
    # name: (mode, B, T, H, Hkv, D, window, positions, dO dtype) - each backward workspace layout
    "fast_stats_in_dq": ("fast", 2, 777, 6, 3, 128, (256, 0), False, torch.bfloat16),
    "fast_fp32_dO_positions": ("fast", 2, 500, 4, 2, 128, (-1, 0), True, torch.float32),
    "exact_window": ("exact", 2, 300, 4, 2, 64, (100, 0), True, torch.float32),
}


@pytest.mark.parametrize("case", sorted(WS_CASES))
def test_backward_ignores_prior_workspace_contents(gpu, case):
    """The gradients depend only on the call's inputs: the same backward with
    its workspace filled beforehand with NaN, with zeros, and with another
    call's contents gives the same bits, and so do calls after a different
    problem has run.  (Every workspace word a kernel reads is written earlier
    in the same call, and every output element has one writer with a fixed
    order of accumulation: no atomics, and the dK/dV work counters only choose
    which workgroup runs an item.)"""
    from femtochat_amd import backward_workspace_bytes, delta_attention_

    mode, B, T, H, Hkv, D, window, with_pos, dtype = WS_CASES[case]
    fast = mode == "fast"
    A = MFMAFast() if fast else MFMAExact()
    Q, K, V, dO = _inputs(23, B, T, H, Hkv, D, fast)
    Qd, Kd, Vd = (_dev(x, fast, gpu) for x in (Q, K, V))
    dOd = torch.from_numpy(dO).to(device=gpu, dtype=dtype)
    pos = torch.from_numpy(W.document_positions(T, B, seed=7, mean=60, sigma=1.0, cap=300)).to(gpu) \
        if with_pos else None
    O, l, m = gpu_forward(A, Qd, Kd, Vd, window, pos, out_dtype=dtype)
    nws = backward_workspace_bytes(A, Qd, Kd, positions=pos, dout_dtype=dtype)
    ws = torch.empty(nws, dtype=torch.uint8, device=gpu)
    gd = dtype if fast else torch.float32
    outs = []
    for fill in ("nan", "zero", "previous", "other"):
        if fill == "nan":
            ws.view(torch.uint8).fill_(0xFF)  # every float word a NaN, every int word -1
        elif fill == "zero":
            ws.zero_()
        elif fill == "other":  # a smaller, different problem through the same workspace first
            o = [x[:1, :200].contiguous() for x in (Qd, Kd, Vd)]
            o_dO = dOd[:1, :200].contiguous()
            oO, ol, om = gpu_forward(A, *o, (-1, 0), out_dtype=dtype)
            g = [torch.zeros(x.shape, dtype=gd, device=gpu) for x in o]
            delta_attention_(A, *g, o_dO, *o, oO, ol, om, (-1, 0), accumulate=False, workspace=ws)
        grads = [torch.full(x.shape, float("nan"), dtype=gd, device=gpu) for x in (Qd, Kd, Vd)]
        delta_attention_(A, *grads, dOd, Qd, Kd, Vd, O, l, m, window, positions=pos, accumulate=False,
                         workspace=ws)
        torch.cuda.synchronize()
        say(f"workspace {fill}: done")
        outs.append(grads)
    for grads in outs[1:]:
        for name, x, y in zip(("dQ", "dK", "dV"), outs[0], grads):
            assert not torch.isnan(y).any(), name
            assert torch.equal(x, y), f"{name} depends on the workspace's prior contents"


def test_cross_mix_statistics_contract(gpu):
    """Oracle forward statistics fed to the GPU backward, and GPU statistics to
    the oracle backward, agree: pins the meaning of l and m across the boundary."""
    A = MFMAExact()
    B, T, H, Hkv, D = 1, 200, 2, 1, 64
    Q, K, V, dO = _inputs(3, B, T, H, Hkv, D, False)
    O_r, l_r, m_r = R.forward(Q, K, V, (-1, 0))
    Qd, Kd, Vd, dOd = (_dev(x, False, gpu) for x in (Q, K, V, dO))
    Od, ld, md = (torch.from_numpy(x.astype(np.float32)).to(gpu) for x in (O_r, l_r, m_r))
    g = gpu_backward(A, dOd, Qd, Kd, Vd, Od, ld, md, (-1, 0))
    g_ref = R.backward(dO, Q, K, V, O_r, l_r, m_r, (-1, 0))
    for x, r in zip(g, g_ref):
        assert rel_err(to_np(x), r) <= 1e-4
    O, l, m = gpu_forward(A, Qd, Kd, Vd, (-1, 0))
    g2 = R.backward(dO, Q, K, V, to_np(O), to_np(l), to_np(m), (-1, 0))
    for x, r in zip(g2, g_ref):
        assert rel_err(x, r) <= 1e-4


def test_gqa_equals_repeated_kv(gpu):
    """GQA == MHA with K/V repeated per group; dK/dV(GQA) = group sums of dK/dV(MHA)."""
    A = MFMAFast()
    B, T, H, Hkv, D = 2, 256, 6, 2, 128
    G = H // Hkv
    Q, K, V, dO = _inputs(5, B, T, H, Hkv, D, True)
    Kr, Vr = np.repeat(K, G, axis=2), np.repeat(V, G, axis=2)
    args = [_dev(x, True, gpu) for x in (Q, K, V, dO, Kr, Vr)]
    Qd, Kd, Vd, dOd, Krd, Vrd = args
    O1, l1, m1 = gpu_forward(A, Qd, Kd, Vd, (-1, 0))
    O2, l2, m2 = gpu_forward(A, Qd, Krd, Vrd, (-1, 0))
    assert torch.equal(O1, O2) and torch.equal(l1, l2) and torch.equal(m1, m2)
    g1 = gpu_backward(A, dOd, Qd, Kd, Vd, O1, l1, m1, (-1, 0), grad_dtype=torch.float32)
    g2 = gpu_backward(A, dOd, Qd, Krd, Vrd, O2, l2, m2, (-1, 0), grad_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(g1[0], g2[0])
    for a, b in zip(g1[1:], g2[1:]):
        summed = to_np(b).reshape(B, T, Hkv, G, D).sum(axis=3)
        assert rel_err(to_np(a), summed) <= 1e-5


def test_document_mask_equals_segments(gpu):
    """A packed row with the document mask equals attention run separately on each
    document (the reference semantics per segment)."""
    A = MFMAExact()
    T, H, Hkv, D = 300, 2, 1, 64
    lengths = [37, 120, 1, 64, 78]
    pos = np.concatenate([np.arange(n, dtype=np.int32) for n in lengths])[None, :]
    Q, K, V, dO = _inputs(9, 1, T, H, Hkv, D, False)
    Qd, Kd, Vd, dOd = (_dev(x, False, gpu) for x in (Q, K, V, dO))
    pos_d = torch.from_numpy(pos).to(gpu)
    O, l, m = gpu_forward(A, Qd, Kd, Vd, (-1, 0), pos_d)
    g = gpu_backward(A, dOd, Qd, Kd, Vd, O, l, m, (-1, 0), pos_d)
    t0 = 0
    for n in lengths:
        sl = slice(t0, t0 + n)
        Os, ls, ms = gpu_forward(A, Qd[:, sl].contiguous(), Kd[:, sl].contiguous(), Vd[:, sl].contiguous(), (-1, 0))
        gs = gpu_backward(A, dOd[:, sl].contiguous(), Qd[:, sl].contiguous(), Kd[:, sl].contiguous(),
                          Vd[:, sl].contiguous(), Os, ls, ms, (-1, 0))
        assert rel_err(to_np(O[:, sl]), to_np(Os)) <= 1e-6
        assert np.max(np.abs(to_np(l[:, :, sl]) - to_np(ls))) <= 1e-5 * max(1.0, float(to_np(ls).max()))
        for a, b in zip(g, gs):
            assert rel_err(to_np(a[:, sl]), to_np(b)) <= 1e-5
        t0 += n


# ---------------------------------------------------------------------------
# Full-size BASELINE workloads.


def _segments(pos_row):
    T = len(pos_row)
    start = np.maximum(0, np.arange(T) - pos_row.astype(np.int64))
    cuts = [0] + [t for t in range(1, T) if start[t] != start[t - 1]] + [T]
    return [(cuts[i], cuts[i + 1]) for i in range(len(cuts) - 1)]


def _oracle_slice(h, b, kv, G, window, O_gpu, l_gpu, m_gpu):
    """Oracle fwd/bwd for batch row b and KV group kv (the group's G query heads)."""
    heads = list(range(kv * G, (kv + 1) * G))
    Q = h.Q[b:b + 1][:, :, heads]
    K = h.K[b:b + 1][:, :, kv:kv + 1]
    V = h.V[b:b + 1][:, :, kv:kv + 1]
    dO = h.dO[b:b + 1][:, :, heads]
    pos = None if h.positions is None else h.positions[b:b + 1]
    Og = O_gpu[b:b + 1][:, :, heads]
    lg = l_gpu[b:b + 1][:, heads]
    mg = m_gpu[b:b + 1][:, heads]
    if pos is not None and np.any(pos[0] != np.arange(pos.shape[1])):
        # Packed documents: the reference attention on each document segment.
        T = Q.shape[1]
        O = np.zeros(Q.shape)
        l = np.zeros((1, len(heads), T))
        m = np.zeros((1, len(heads), T))
        dQ, dK, dV = np.zeros(Q.shape), np.zeros(K.shape), np.zeros(V.shape)
        for s, e in _segments(pos[0]):
            o, ll, mm = R.forward(Q[:, s:e], K[:, s:e], V[:, s:e], window)
            O[:, s:e], l[:, :, s:e], m[:, :, s:e] = o, ll, mm
            gq, gk, gv = R.backward(dO[:, s:e], Q[:, s:e], K[:, s:e], V[:, s:e], Og[:, s:e], lg[:, :, s:e],
                                    mg[:, :, s:e], window)
            dQ[:, s:e], dK[:, s:e], dV[:, s:e] = gq, gk, gv
        return (O, l, m), (dQ, dK, dV)
    fwd = R.forward(Q, K, V, window, pos)
    bwd = R.backward(dO, Q, K, V, Og, lg, mg, window, pos)
    return fwd, bwd


# The identities hold to the rounding of P (bf16 in fast mode, before P.V and
# dS) and of the stored gradients.
# (measured: 1e-7 to 4e-7 exact, 2e-4 to 6e-4 fast, on C1..C5; a dropped tile
# moves them by about its share of the keys, 1e-2 and more)
IDENTITY_TOL = {"exact": 1e-5, "fast": 4e-3}
# Scale identity |<dQ,Q> - <dK,K>| / (sum|dQ Q| + sum|dK K|) per (batch, KV
# group): the rounding of dS to bf16 (fast) or fp32 noise (exact); a dropped
# block of dQ or dK moves it by 1e-4 and more (tests/test_oracle.py).
SCALE_TOL = {"exact": 1e-5, "fast": 1e-2}


def _units(B, Hkv):
    """(batch, KV group) units whose grid row b*Hkv + kv covers every residue
    mod 8, plus the first, the last and a middle batch row."""
    n = B * Hkv
    picks = {0, n - 1, (B // 2) * Hkv + Hkv // 2}
    if n >= 8:
        span = n // 8
        picks |= {r + 8 * ((3 * r + 1) % span) for r in range(8)}
    else:
        picks |= set(range(n))
    return sorted((u // Hkv, u % Hkv) for u in picks if u < n)


def _scale_identity(dQ, Q, dK, K, G):
    B, T, H, D = Q.shape
    Hkv = K.shape[2]
    qq = (dQ.double() * Q.double()).reshape(B, T, Hkv, G, D)
    kk = dK.double() * K.double()
    num = (qq.sum(dim=(1, 3, 4)) - kk.sum(dim=(1, 3))).abs()
    den = qq.abs().sum(dim=(1, 3, 4)) + kk.abs().sum(dim=(1, 3))
    return (num / den.clamp_min(1e-300)).max().item()


def _single_key_rows(h, window):
    """(b, q) of every query that sees exactly one key (itself): the first
    query of a row and, with positions, every document start."""
    out = []
    B, T = h.Q.shape[0], h.Q.shape[1]
    for b in range(B):
        qs = [0] if h.positions is None else list(np.nonzero(h.positions[b] == 0)[0]) + [0]
        for q in sorted(set(int(x) for x in qs)):
            vis = R.visible(T, window, None if h.positions is None else h.positions[b])[q]
            if vis.sum() == 1 and vis[q]:
                out.append((b, q))
    return out


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4", "C5"])
def test_baseline_workload(gpu, name):
    wl = W.WORKLOADS[name]
    A = MFMAFast() if wl.mode == "fast" else MFMAExact()
    tol = TOL[wl.mode]
    G = wl.H // wl.Hkv
    for layer in range(wl.layers):
        say(f"workload {name} layer {layer} window {wl.windows[layer]}")
        h = W.host_inputs(wl, layer)
        dt = torch.bfloat16 if wl.mode == "fast" else torch.float32
        Qd, Kd, Vd, dOd = (torch.from_numpy(x).to(gpu, dt).contiguous() for x in (h.Q, h.K, h.V, h.dO))
        pos_d = None if h.positions is None else torch.from_numpy(h.positions).to(gpu)
        O, l, m = gpu_forward(A, Qd, Kd, Vd, h.window, pos_d)
        dQ, dK, dV = gpu_backward(A, dOd, Qd, Kd, Vd, O, l, m, h.window, pos_d)
        torch.cuda.synchronize()
        On, ln, mn = to_np(O), to_np(l), to_np(m)
        gn = [to_np(x) for x in (dQ, dK, dV)]
        assert all(np.isfinite(x).all() for x in [On, ln, mn] + gn)
        # Properties over the whole output: every query sees at least itself.
        assert (ln >= 1.0 - 1e-6).all()
        # Every query's probabilities sum to one over its visible keys and its
        # dS row sums to zero, so per (batch, KV head), over all tokens:
        # sum dV = the sum of the group's dO, and sum dK = 0 (relative to the
        # sum of |dK|).  Any tile dropped or counted twice breaks them.
        dO_sum = dOd.double().reshape(wl.B, wl.T, wl.Hkv, G, wl.D).sum(dim=(1, 3))
        eV = ((dV.double().sum(dim=1) - dO_sum).abs().max() / dO_sum.abs().max()).item()
        eK = (dK.double().sum(dim=1).abs() / dK.double().abs().sum(dim=1).clamp_min(1e-30)).max().item()
        say(f"  sum dV vs sum dO {eV:.2e}, |sum dK| / sum |dK| {eK:.2e}")
        assert eV <= IDENTITY_TOL[wl.mode] and eK <= IDENTITY_TOL[wl.mode]
        eS = _scale_identity(dQ, Qd, dK, Kd, G)
        say(f"  scale identity <dQ,Q> - <dK,K> {eS:.2e}")
        assert eS <= SCALE_TOL[wl.mode]
        # Rows whose query sees a single key, over every (batch, head).
        rows1 = _single_key_rows(h, h.window)
        assert rows1, "every row's first query sees one key"
        bi = np.array([r[0] for r in rows1])
        qi = np.array([r[1] for r in rows1])
        kvh = np.arange(wl.H) // G
        Vsel = h.V[bi, qi][:, kvh]  # (n, H, D)
        Osel = On[bi, qi]
        tau = 1.0 / np.sqrt(wl.D)
        m_ref = tau * np.einsum("nhd,nhd->nh", h.Q[bi, qi].astype(np.float64), h.K[bi, qi][:, kvh].astype(np.float64))
        assert np.max(np.abs(Osel - Vsel)) <= 1e-6 * max(1.0, float(np.abs(Vsel).max())), "O = V at single-key rows"
        assert np.all(np.abs(ln[bi, :, qi] - 1.0) <= 1e-6), "l = 1 at single-key rows"
        assert np.max(np.abs(mn[bi, :, qi] - m_ref) / np.maximum(1.0, np.abs(m_ref))) <= 1e-5, "m = tau q.k"
        dq1 = np.abs(gn[0][bi, qi]).max()
        assert dq1 <= 1e-5 * max(float(np.abs(gn[0]).max()), 1e-30), f"dQ = 0 at single-key rows ({dq1})"
        say(f"  {len(rows1)} single-key rows x {wl.H} heads: O = V, l = 1, m = tau q.k, dQ = 0")
        for b, kv in _units(wl.B, wl.Hkv):
            heads = list(range(kv * G, (kv + 1) * G))
            (O_r, l_r, m_r), (dQ_r, dK_r, dV_r) = _oracle_slice(h, b, kv, G, h.window, On, ln, mn)
            eO = rel_err(On[b:b + 1][:, :, heads], O_r)
            eL = lse_err(ln[b:b + 1][:, heads], mn[b:b + 1][:, heads], l_r, m_r)
            e = [rel_err(gn[0][b:b + 1][:, :, heads], dQ_r), rel_err(gn[1][b:b + 1][:, :, kv:kv + 1], dK_r),
                 rel_err(gn[2][b:b + 1][:, :, kv:kv + 1], dV_r)]
            say(f"  b={b} kv={kv}: O {eO:.2e} LSE {eL:.2e} dQ {e[0]:.2e} dK {e[1]:.2e} dV {e[2]:.2e}")
            assert eO <= tol and eL <= TOL_LSE and max(e) <= tol


@pytest.mark.parametrize("name,layer", [("C2", 0), ("C3", 0), ("C4", 0)])
def test_full_output_against_blocked_restatement(gpu, name, layer):
    """Every (batch, KV group) of a full-size workload against the reference's
    blocked algorithm restated in float32 with BLAS products
    (oracle/fa1_blas.py, pinned to the float64 oracle in tests/test_oracle.py;
    a few seconds on the host's BLAS threads for a whole C3 batch): O and the
    log-sum-exp from the same inputs, and the gradients from the GPU's own O,
    l, m on both sides, at the contract's tolerances, unit by unit."""
    from oracle import fa1_blas

    wl = W.WORKLOADS[name]
    A = MFMAFast() if wl.mode == "fast" else MFMAExact()
    tol = TOL[wl.mode]
    G = wl.H // wl.Hkv
    h = W.host_inputs(wl, layer)
    say(f"full output {name} layer {layer} window {h.window}: B={wl.B} T={wl.T} H={wl.H} Hkv={wl.Hkv}")
    dt = torch.bfloat16 if wl.mode == "fast" else torch.float32
    Qd, Kd, Vd, dOd = (torch.from_numpy(x).to(gpu, dt).contiguous() for x in (h.Q, h.K, h.V, h.dO))
    pos_d = None if h.positions is None else torch.from_numpy(h.positions).to(gpu)
    O, l, m = gpu_forward(A, Qd, Kd, Vd, h.window, pos_d)
    dQ, dK, dV = gpu_backward(A, dOd, Qd, Kd, Vd, O, l, m, h.window, pos_d)
    torch.cuda.synchronize()
    On, ln, mn = to_np(O), to_np(l), to_np(m)
    gn = [to_np(x) for x in (dQ, dK, dV)]
    f32 = [np.ascontiguousarray(x, dtype=np.float32) for x in (h.Q, h.K, h.V, h.dO)]
    O_r, l_r, m_r = fa1_blas.forward(f32[0], f32[1], f32[2], h.window, h.positions)
    g_r = fa1_blas.backward(f32[3], f32[0], f32[1], f32[2], On, ln, mn, h.window, h.positions)
    say("  restatement done")
    worst = [0.0] * 5
    for b in range(wl.B):
        for kv in range(wl.Hkv):
            heads = slice(kv * G, (kv + 1) * G)
            e = [rel_err(On[b, :, heads], O_r[b, :, heads]),
                 lse_err(ln[b, heads], mn[b, heads], l_r[b, heads], m_r[b, heads]),
                 rel_err(gn[0][b, :, heads], g_r[0][b, :, heads]),
                 rel_err(gn[1][b, :, kv], g_r[1][b, :, kv]),
                 rel_err(gn[2][b, :, kv], g_r[2][b, :, kv])]
            worst = [max(w, x) for w, x in zip(worst, e)]
    say(f"  worst over {wl.B * wl.Hkv} units: O {worst[0]:.2e} LSE {worst[1]:.2e} dQ {worst[2]:.2e} "
        f"dK {worst[3]:.2e} dV {worst[4]:.2e}")
    assert worst[0] <= tol and worst[1] <= TOL_LSE and max(worst[2:]) <= tol


GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.mark.parametrize("name", ["c1_golden.npz", "slice_golden.npz"])
def test_golden_fixtures(gpu, name):
    # The committed fixtures (tests/golden/make_golden.py): C1 in exact mode,
    # the document-masked C3 slice (bf16 inputs) in fast mode.
    z = np.load(GOLDEN / name)
    fast = name.startswith("slice")
    mode = "fast" if fast else "exact"
    A = MFMAFast() if fast else MFMAExact()
    window = tuple(int(w) for w in z["window"])
    say(f"golden {name} window {window}")
    Qd, Kd, Vd, dOd = (_dev(z[k], fast, gpu) for k in ("Q", "K", "V", "dO"))
    pos_d = torch.from_numpy(z["positions"].astype(np.int32)).to(gpu)
    O, l, m = gpu_forward(A, Qd, Kd, Vd, window, pos_d)
    dQ, dK, dV = gpu_backward(A, dOd, Qd, Kd, Vd, O, l, m, window, pos_d)
    torch.cuda.synchronize()
    tol = TOL[mode]
    assert rel_err(to_np(O), z["O"]) <= tol
    assert lse_err(to_np(l), to_np(m), z["l"], z["m"]) <= TOL_LSE
    for k, x in (("dQ", dQ), ("dK", dK), ("dV", dV)):
        assert rel_err(to_np(x), z[k]) <= tol, k


@pytest.mark.parametrize("growth", [40.0, 140.0])
def test_fast_forward_large_logit_growth(gpu, growth):
    # Scores rise along the keys so that, for late queries, the last key's
    # log2-scaled score exceeds the first key block's by about `growth`.  At
    # 40 the fast forward runs with probabilities up to 2^40 against its
    # reference; at 140 it passes its 2^64 limit and the wave recomputes its
    # rows with the exact maximum first.  Either way the outputs must match.
    B, T, H, Hkv, D = 1, 200, 2, 1, 64
    rng = np.random.Generator(np.random.PCG64(int(growth)))
    c2 = np.log2(np.e) / np.sqrt(D)
    beta = growth / (c2 * 2.0 * D) * (np.arange(T) / T)
    Q = (2.0 + 0.05 * rng.standard_normal((B, T, H, D))).astype(np.float32)
    K = (beta[None, :, None, None] + 0.05 * rng.standard_normal((B, T, Hkv, D))).astype(np.float32)
    V = rng.standard_normal((B, T, Hkv, D)).astype(np.float32)
    dO = (0.1 * rng.standard_normal((B, T, H, D))).astype(np.float32)
    Q, K, V, dO = (torch.from_numpy(x).bfloat16().float().numpy() for x in (Q, K, V, dO))
    Qd, Kd, Vd = (_dev(x, True, gpu) for x in (Q, K, V))
    say(f"case large logit growth {growth}")
    O, l, m = gpu_forward(MFMAFast(), Qd, Kd, Vd, (-1, 0))
    torch.cuda.synchronize()
    O_ref, l_ref, m_ref = R.forward(Q, K, V, (-1, 0))
    assert np.all(np.isfinite(to_np(O))) and np.all(np.isfinite(to_np(l)))
    assert rel_err(to_np(O), O_ref) <= TOL["fast"]
    # L reaches ~100 here, so the float32 statistics carry ~1e-5 absolute
    # rounding: the bound is relative to |L|.
    L = to_np(m).astype(np.float64) + np.log(to_np(l).astype(np.float64))
    L_ref = m_ref + np.log(l_ref)
    assert np.max(np.abs(L - L_ref) / np.maximum(1.0, np.abs(L_ref))) <= TOL_LSE
    dOd = _dev(dO, True, gpu)
    grads = gpu_backward(MFMAFast(), dOd, Qd, Kd, Vd, O, l, m, (-1, 0))
    torch.cuda.synchronize()
    # Keys here share a common component near 6 and dS sums to zero along a
    # row, so at growth 140 fast mode's bf16 rounding of dS (as the
    # reference's) leaves a few percent in dQ against the unrounded float64
    # oracle; the oracle that rounds P and dS as the reference's tensor-core
    # backward does is the one to match.
    g_ref = R.backward(dO, Q, K, V, to_np(O), to_np(l), to_np(m), (-1, 0), fast=growth > 64)
    for name, x, r in zip(("dQ", "dK", "dV"), grads, g_ref):
        e = rel_err(to_np(x), r)
        say(f"  {name} rel err {e:.2e}")
        assert e <= TOL["fast"], name


@pytest.mark.parametrize("mode", ["exact", "fast"])
@pytest.mark.parametrize("D", [64, 128])
def test_nan_query_stays_in_its_row(gpu, mode, D):
    # A NaN in one query makes that query's scores NaN.  The reference's
    # maximum, exp and sums carry it (Julia's max propagates NaN), so that row's
    # O and log-sum-exp are NaN; the other queries never see it and must match
    # the oracle on the clean input.
    fast = mode == "fast"
    B, T, H, Hkv = 1, 200, 2, 1
    bad_t, bad_h = 150, 1
    Q, K, V, _ = _inputs(11 + D, B, T, H, Hkv, D, fast)
    Qn = Q.copy()
    Qn[0, bad_t, bad_h, 3] = np.nan
    Qd, Kd, Vd = (_dev(x, fast, gpu) for x in (Qn, K, V))
    say(f"case NaN query mode={mode} D={D} at t={bad_t} h={bad_h}")
    O, l, m = gpu_forward(MFMAFast() if fast else MFMAExact(), Qd, Kd, Vd, (-1, 0))
    torch.cuda.synchronize()
    O, l, m = to_np(O).copy(), to_np(l).copy(), to_np(m).copy()
    assert np.all(np.isnan(O[0, bad_t, bad_h])), "the NaN query's output row must be NaN"
    assert np.isnan(l[0, bad_h, bad_t]) or np.isnan(m[0, bad_h, bad_t]), "its log-sum-exp must be NaN"
    O_ref, l_ref, m_ref = R.forward(Q, K, V, (-1, 0))
    O[0, bad_t, bad_h] = O_ref[0, bad_t, bad_h]
    l[0, bad_h, bad_t], m[0, bad_h, bad_t] = l_ref[0, bad_h, bad_t], m_ref[0, bad_h, bad_t]
    assert np.all(np.isfinite(O)) and np.all(np.isfinite(l))
    assert rel_err(O, O_ref) <= TOL[mode]
    assert lse_err(l, m, l_ref, m_ref) <= TOL_LSE


@pytest.fixture(scope="module")
def c5_gpu_outputs(gpu):
    wl = W.WORKLOADS["C5"]
    h = W.host_inputs(wl, 0)
    say(f"C5 full output: B={wl.B} T={wl.T} H={wl.H} Hkv={wl.Hkv}")
    Qd, Kd, Vd, dOd = (torch.from_numpy(x).to(gpu, torch.bfloat16).contiguous() for x in (h.Q, h.K, h.V, h.dO))
    pos_d = torch.from_numpy(h.positions).to(gpu)
    A = MFMAFast()
    O, l, m = gpu_forward(A, Qd, Kd, Vd, h.window, pos_d)
    dQ, dK, dV = gpu_backward(A, dOd, Qd, Kd, Vd, O, l, m, h.window, pos_d)
    torch.cuda.synchronize()
    return wl, h, [to_np(x) for x in (O, l, m, dQ, dK, dV)]


@pytest.mark.parametrize("b", [0, 1, 2, 3])
def test_c5_full_output_by_documents(c5_gpu_outputs, b):
    """C5 (packed documents, T = 8192) over every KV group of batch row b,
    against the float64 oracle run document by document (attention never
    crosses a document start, so each segment is an independent causal
    problem): O, the log-sum-exp and the gradients from the GPU's own O, l, m,
    unit by unit, at the contract's tolerances."""
    wl, h, (On, ln, mn, gq, gk, gv) = c5_gpu_outputs
    G = wl.H // wl.Hkv
    worst = [0.0] * 5
    for kv in range(wl.Hkv):
        (O_r, l_r, m_r), (dq_r, dk_r, dv_r) = _oracle_slice(h, b, kv, G, h.window, On, ln, mn)
        heads = slice(kv * G, (kv + 1) * G)
        e = [rel_err(On[b:b + 1, :, heads], O_r), lse_err(ln[b:b + 1, heads], mn[b:b + 1, heads], l_r, m_r),
             rel_err(gq[b:b + 1, :, heads], dq_r), rel_err(gk[b:b + 1, :, kv:kv + 1], dk_r),
             rel_err(gv[b:b + 1, :, kv:kv + 1], dv_r)]
        worst = [max(w, x) for w, x in zip(worst, e)]
    say(f"  C5 row {b}, {wl.Hkv} units: O {worst[0]:.2e} LSE {worst[1]:.2e} dQ {worst[2]:.2e} dK {worst[3]:.2e} "
        f"dV {worst[4]:.2e}")
    assert worst[0] <= TOL["fast"] and worst[1] <= TOL_LSE and max(worst[2:]) <= TOL["fast"]
