"""fc_attn_bwd_noalloc, the backward entry point that allocates nothing and
takes its workspace from the library's per-GPU scratch array, against
fc_attn_bwd with a caller-owned workspace: the same kernels, so the gradients
must be bit-identical.  Two calls in a row, the second on a smaller problem
(the scratch then still holds the first call's contents), in every workspace
layout the backward has: fast mode with an fp32 dO (bf16 copy of dO in the
scratch) and document positions (per-chunk key bounds in the scratch), fast
mode with bf16 O and dO (statistics computed by the dQ kernel), exact mode
with a sliding window; adding into non-zero gradients as well as writing."""
import ctypes

import numpy as np
import pytest
import torch

from femtochat_amd import MFMAExact, MFMAFast, _lib
from femtochat_amd import kernels as Kn
from tests.helpers import gpu_forward, say

pytestmark = pytest.mark.gpu


def _positions(B, T, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    pos = np.zeros((B, T), np.int32)
    for b in range(B):
        t = 0
        while t < T:
            n = int(rng.integers(1, max(2, T // 3)))
            pos[b, t:t + n] = np.arange(min(n, T - t))
            t += n
    return pos


def _problem(gpu, mode, B, T, H, Hkv, D, window, with_pos, io_dtype, grad_dtype, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    in_dtype = torch.bfloat16 if mode == "fast" else torch.float32
    Q = torch.randn(B, T, H, D, device=gpu, generator=g).to(in_dtype)
    K = torch.randn(B, T, Hkv, D, device=gpu, generator=g).to(in_dtype)
    V = torch.randn(B, T, Hkv, D, device=gpu, generator=g).to(in_dtype)
    pos = torch.from_numpy(_positions(B, T, seed)).to(gpu) if with_pos else None
    A = MFMAFast() if mode == "fast" else MFMAExact()
    O, l, m = gpu_forward(A, Q, K, V, window, pos, out_dtype=io_dtype)
    dO = (0.1 * torch.randn(B, T, H, D, device=gpu, generator=g)).to(io_dtype)
    init = [0.01 * torch.randn(x.shape, device=gpu, generator=g).to(grad_dtype) for x in (Q, K, V)]
    return A, dict(Q=Q, K=K, V=V, O=O, l=l, m=m, dO=dO, pos=pos, init=init, window=window)


def _run(entry, A, p, accumulate):
    gd = p["init"][0].dtype
    dQ, dK, dV = (x.clone() if accumulate else torch.full_like(x, float("nan")) for x in p["init"])
    d = Kn._desc(A, p["Q"], p["K"], p["window"], Kn._dtype_code(p["O"].dtype), Kn._dtype_code(p["dO"].dtype),
                 Kn._dtype_code(gd), overwrite=not accumulate)
    lib = _lib.lib()
    dev = p["Q"].device
    args = [ctypes.byref(d)] + [Kn._ptr(p[k]) for k in ("dO", "Q", "K", "V", "O", "l", "m", "pos")] + \
        [Kn._ptr(dQ), Kn._ptr(dK), Kn._ptr(dV)]
    if entry == "noalloc":
        st = lib.fc_attn_bwd_noalloc(*args, Kn._stream_ptr(dev))
    else:
        n = ctypes.c_size_t(0)
        _lib.check(lib.fc_attn_workspace_bytes(ctypes.byref(d), _lib.FC_PASS_BACKWARD, int(p["pos"] is not None),
                                               ctypes.byref(n)))
        ws = torch.empty(int(n.value) + 256, dtype=torch.uint8, device=dev)
        aligned = (ws.data_ptr() + 255) & ~255
        st = lib.fc_attn_bwd(*args, ctypes.c_void_p(aligned), ctypes.c_size_t(int(n.value)), Kn._stream_ptr(dev))
        torch.cuda.synchronize()
        del ws
    _lib.check(st)
    torch.cuda.synchronize()
    return dQ, dK, dV


CASES = {
    # name: (mode, first problem, second (smaller) problem, O/dO dtype, gradient dtype)
    "fast_fp32_dO_positions": ("fast", (2, 1000, 8, 4, 128, (-1, 0), True), (1, 333, 4, 2, 64, (-1, 0), True),
                               torch.float32, torch.float32),
    "fast_bf16_stats_in_dq": ("fast", (2, 777, 6, 3, 128, (256, 0), False), (1, 129, 2, 1, 128, (-1, 0), False),
                              torch.bfloat16, torch.bfloat16),
    "exact_window": ("exact", (2, 600, 4, 2, 64, (100, 0), True), (1, 65, 2, 2, 32, (-1, 0), False),
                     torch.float32, torch.float32),
}


@pytest.mark.parametrize("accumulate", [False, True])
@pytest.mark.parametrize("case", sorted(CASES))
def test_noalloc_matches_workspace_entry_point(gpu, case, accumulate):
    mode, first, second, io_dtype, grad_dtype = CASES[case]
    for i, shape in enumerate((first, second)):
        B, T, H, Hkv, D, window, with_pos = shape
        say(f"noalloc case={case} call={i} accumulate={accumulate} B={B} T={T} H={H} Hkv={Hkv} D={D} "
            f"window={window} pos={with_pos}")
        A, p = _problem(gpu, mode, B, T, H, Hkv, D, window, with_pos, io_dtype, grad_dtype, seed=17 + i)
        want = _run("workspace", A, p, accumulate)
        got = _run("noalloc", A, p, accumulate)
        for name, a, b in zip(("dQ", "dK", "dV"), got, want):
            assert not torch.isnan(b).any(), f"{name}: the workspace entry point left NaN"
            assert torch.equal(a, b), f"call {i}: {name} differs from fc_attn_bwd (max |diff| " \
                f"{(a.float() - b.float()).abs().max().item():.3e})"

