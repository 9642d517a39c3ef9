"""The XLA FFI callbacks (include/femtochat_xla.h).

CPU: binding validates descriptors on the host, returns a distinct callback
per call site and reports the backward's workspace size (the library's need
plus 255 bytes of alignment slack); the pool of 256 call sites is exhausted
cleanly (in a subprocess, so this process keeps its slots).  GPU: each
callback, invoked with a stream and the buffers in XLA's order (inputs, then
outputs), matches the float64 oracle within the fast-mode tolerance, also
with its workspace at a 64-byte (not 256-byte) boundary as XLA allocates it,
and writes the same bits as the direct C entry points for the same call; the
embedding callbacks match torch's embedding and its gradient.
"""
from __future__ import annotations

import ctypes
import subprocess
import sys
from pathlib import Path

import pytest
import torch

import femtochat_amd._lib as L
from femtochat_amd import MFMAFast, attention_, delta_attention_, embedding, embedding_gradient_
from femtochat_amd.kernels import _desc, _stream_ptr
from oracle import attention_ref as R
from tests.helpers import TOL, TOL_LSE, lse_err, rel_err, to_np

ROOT = Path(__file__).resolve().parents[1]


def _attn_desc(B=2, T=40, H=4, Hkv=2, D=64, window=(-1, 0)):
    Q = torch.empty(B, T, H, D, dtype=torch.bfloat16)
    K = torch.empty(B, T, Hkv, D, dtype=torch.bfloat16)
    return _desc(MFMAFast(), Q, K, window, L.FC_BF16, L.FC_BF16, L.FC_BF16)


def _embed_desc(D=32, vocab=50, N=12):
    d = L.EmbedDesc()
    d.D, d.vocab, d.N, d.index_base, d.index_type, d.y_dtype, d.flags = D, vocab, N, 0, L.FC_INDEX_I32, L.FC_F32, 0
    return d


def _callback(ptr):
    assert ptr, L.lib().fc_xla_last_error().decode()
    return L.XLA_CALLBACK(ptr)


def _buffers(*tensors):
    return (ctypes.c_void_p * len(tensors))(*[t.data_ptr() for t in tensors])


def test_binding_validates_and_returns_distinct_callbacks():
    lib = L.lib()
    a = lib.fc_xla_bind_attention_fwd(ctypes.byref(_attn_desc()), 0)
    b = lib.fc_xla_bind_attention_fwd(ctypes.byref(_attn_desc()), 0)
    assert a and b and a != b
    bad = _attn_desc(H=3, Hkv=2)
    assert not lib.fc_xla_bind_attention_fwd(ctypes.byref(bad), 0)
    assert "multiple" in lib.fc_xla_last_error().decode()
    # head_dim 96 runs on padded copies in a workspace, which the forward call site lacks;
    # its backward call site declares the (larger) workspace and binds
    assert not lib.fc_xla_bind_attention_fwd(ctypes.byref(_attn_desc(D=96)), 0)
    assert "padded" in lib.fc_xla_last_error().decode()
    n96 = ctypes.c_size_t(0)
    assert lib.fc_xla_bind_attention_bwd(ctypes.byref(_attn_desc(D=96)), 0, ctypes.byref(n96)) and n96.value > 0
    n = ctypes.c_size_t(0)
    assert lib.fc_xla_bind_attention_bwd(ctypes.byref(_attn_desc()), 1, ctypes.byref(n))
    ref = ctypes.c_size_t(0)
    d = _attn_desc()
    d.flags = L.FC_FLAG_OVERWRITE
    assert lib.fc_attn_workspace_bytes(ctypes.byref(d), L.FC_PASS_BACKWARD, 1, ctypes.byref(ref)) == 0
    assert ref.value > 0 and n.value == ref.value + 255
    assert not lib.fc_xla_bind_attention_bwd(ctypes.byref(_attn_desc()), 0, None)
    e = _embed_desc()
    assert lib.fc_xla_bind_embedding_fwd(ctypes.byref(e)) and lib.fc_xla_bind_embedding_bwd(ctypes.byref(e))
    e.y_dtype = 9
    assert not lib.fc_xla_bind_embedding_fwd(ctypes.byref(e))
    assert "invalid embedding" in lib.fc_xla_last_error().decode()


def test_slot_pool_is_exhausted_cleanly():
    code = (
        "import ctypes, femtochat_amd._lib as L\n"
        "from tests.test_xla_bridge import _embed_desc\n"
        "lib = L.lib(); d = _embed_desc()\n"
        "ptrs = [lib.fc_xla_bind_embedding_fwd(ctypes.byref(d)) for _ in range(257)]\n"
        "assert all(ptrs[:256]) and len(set(ptrs[:256])) == 256, 'first 256 bind'\n"
        "assert not ptrs[256] and '256' in lib.fc_xla_last_error().decode()\n"
        "print('ok')\n"
    )
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "ok" in r.stdout, r.stderr


@pytest.mark.gpu
def test_attention_callbacks_match_the_oracle(gpu):
    B, T, H, Hkv, D = 2, 40, 4, 2, 64
    g = torch.Generator(device=gpu).manual_seed(1)
    Q = torch.randn(B, T, H, D, device=gpu, generator=g).to(torch.bfloat16)
    K = torch.randn(B, T, Hkv, D, device=gpu, generator=g).to(torch.bfloat16)
    V = torch.randn(B, T, Hkv, D, device=gpu, generator=g).to(torch.bfloat16)
    dO = torch.randn(B, T, H, D, device=gpu, generator=g).to(torch.bfloat16)
    pos = torch.tensor([list(range(15)) + list(range(25)), list(range(40))], dtype=torch.int32, device=gpu)
    stream = _stream_ptr(gpu)
    tol = TOL["fast"]
    for positions in (None, pos):
        has = positions is not None
        pos_np = positions.cpu().numpy() if has else None
        fwd = _callback(L.lib().fc_xla_bind_attention_fwd(ctypes.byref(_attn_desc(B, T, H, Hkv, D)), int(has)))
        O2, l2, m2 = torch.empty_like(Q), torch.empty(B, H, T, device=gpu), torch.empty(B, H, T, device=gpu)
        ins = (Q, K, V) + ((positions,) if has else ())
        assert fwd(stream, _buffers(*ins, O2, l2, m2))
        n = ctypes.c_size_t(0)
        bwd = _callback(L.lib().fc_xla_bind_attention_bwd(ctypes.byref(_attn_desc(B, T, H, Hkv, D)), int(has),
                                                          ctypes.byref(n)))
        assert n.value > 255
        # XLA's buffers are 64-byte aligned: hand the callback a workspace that
        # starts 64 bytes past a 256-byte boundary.
        arena = torch.empty(n.value + 512, dtype=torch.uint8, device=gpu)
        start = (-arena.data_ptr()) % 256 + 64
        ws = arena[start:start + n.value]
        assert ws.data_ptr() % 256 == 64
        dQ2, dK2, dV2 = torch.full_like(Q, 3), torch.full_like(K, 3), torch.full_like(V, 3)  # overwritten
        assert bwd(stream, _buffers(dO, Q, K, V, O2, l2, m2, *((positions,) if has else ()), dQ2, dK2, dV2, ws)), \
            L.lib().fc_xla_last_error().decode()
        torch.cuda.synchronize()

        q, k, v, do = (to_np(x) for x in (Q, K, V, dO))
        O_ref, l_ref, m_ref = R.forward(q, k, v, (-1, 0), pos_np)
        assert rel_err(to_np(O2), O_ref) <= tol
        assert lse_err(to_np(l2), to_np(m2), l_ref, m_ref) <= TOL_LSE
        g_ref = R.backward(do, q, k, v, to_np(O2), to_np(l2), to_np(m2), (-1, 0), pos_np)
        for name, x, r in zip(("dQ", "dK", "dV"), (dQ2, dK2, dV2), g_ref):
            assert rel_err(to_np(x), r) <= tol, name

        # The same bits as the direct entry points for the same call.
        A = MFMAFast()
        O, l, m = torch.empty_like(Q), torch.empty_like(l2), torch.empty_like(m2)
        attention_(A, O, l, m, Q, K, V, (-1, 0), positions=positions)
        dQ, dK, dV = torch.full_like(Q, 7), torch.full_like(K, 7), torch.full_like(V, 7)
        delta_attention_(A, dQ, dK, dV, dO, Q, K, V, O, l, m, (-1, 0), positions=positions, accumulate=False)
        torch.cuda.synchronize()
        assert torch.equal(O, O2) and torch.equal(l, l2) and torch.equal(m, m2)
        assert torch.equal(dQ, dQ2) and torch.equal(dK, dK2) and torch.equal(dV, dV2)


@pytest.mark.gpu
def test_embedding_callbacks_match_the_direct_calls(gpu):
    D, vocab, N = 32, 50, 12
    g = torch.Generator(device=gpu).manual_seed(2)
    W = torch.randn(vocab, D, device=gpu, generator=g)
    tok = torch.randint(0, vocab, (N,), device=gpu, generator=g, dtype=torch.int32)
    tok[:4] = 5
    dy = torch.randn(N, D, device=gpu, generator=g)
    stream = _stream_ptr(gpu)
    fwd = _callback(L.lib().fc_xla_bind_embedding_fwd(ctypes.byref(_embed_desc(D, vocab, N))))
    bwd = _callback(L.lib().fc_xla_bind_embedding_bwd(ctypes.byref(_embed_desc(D, vocab, N))))
    y = torch.empty(N, D, device=gpu)
    assert fwd(stream, _buffers(W, tok, y))
    dW = torch.full_like(W, 9.0)  # zeroed by the callback first
    assert bwd(stream, _buffers(dy, W, tok, y, dW))
    ref = torch.zeros_like(W)
    embedding_gradient_(ref, dy[4:], tok[4:])
    torch.cuda.synchronize()
    assert torch.equal(y, embedding(W, tok))
    assert torch.equal(y, torch.nn.functional.embedding(tok.long(), W))
    expect = ref.double()
    expect[5] += dy[:4].double().sum(0)
    # (repeated tokens are summed by atomics in no fixed order)
    assert torch.allclose(dW.double(), expect, rtol=1e-6, atol=1e-6)
