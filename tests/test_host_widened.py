"""Host-side checks of the prologue, loss and optimizer mirrors (CPU only:
nothing is launched).  Each refuses CPU tensors (there is no CPU path) and
malformed arguments before reaching the library."""
from __future__ import annotations

import pytest
import torch

import femtochat_amd as F
from femtochat_amd import optim as Fo


def test_prologue_tables_and_cpu_refusal():
    sin, cos = F.rotary_embeddings(12, 32)
    assert sin.shape == (12, 16) and cos.dtype == torch.float32
    with pytest.raises(ValueError):
        F.rotary_embeddings(4, 31)
    with pytest.raises(ValueError, match="no CPU path"):
        F.attention_prologue(torch.zeros(1, 4, 2, 32), (sin, cos))


def test_loss_mirrors_refuse_cpu_and_bad_arguments():
    logits, targets = torch.zeros(3, 10), torch.zeros(3, dtype=torch.int32)
    with pytest.raises(ValueError, match="no CPU path"):
        F.cross_entropy(logits, targets)
    with pytest.raises(ValueError, match="reduction"):
        F.cross_entropy(logits, targets, reduction="max")
    with pytest.raises(ValueError, match="leading shape"):
        F.cross_entropy(logits, torch.zeros(4, dtype=torch.int32))
    with pytest.raises(ValueError, match="no CPU path"):
        F.embedding(torch.zeros(10, 4), targets)
    with pytest.raises(ValueError, match="no CPU path"):
        F.valid_target_count(targets)


def test_optimizer_mirrors_refuse_cpu_and_bad_arguments():
    theta = torch.zeros(8)
    with pytest.raises(ValueError, match="no CPU path"):
        F.AdamW(theta)
    with pytest.raises(TypeError, match="float32"):
        F.AdamW(torch.zeros(8, dtype=torch.float64))
    with pytest.raises(ValueError, match="no CPU path"):
        F.polar_express(torch.zeros(1, 4, 4))
    with pytest.raises(ValueError, match="stack"):
        Fo._polar_desc(torch.zeros(4, 4), 5)
    with pytest.raises(ValueError, match="compute_type"):
        Fo._polar_desc(torch.zeros(1, 4, 4), 5, torch.float16)
    d = Fo._polar_desc(torch.zeros(3, 6, 5), 5, torch.bfloat16)  # torch (k, n, m) = Julia (m, n, k)
    assert (d.m, d.n, d.count, d.steps, d.dtype) == (5, 6, 3, 5, 1)


def test_polar_workspace_sizes():
    import femtochat_amd._lib as L
    import ctypes
    n32, n16 = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert L.lib().fc_polar_workspace_bytes(ctypes.byref(L.PolarDesc(512, 2048, 8, 5, 0)), ctypes.byref(n32)) == 0
    assert L.lib().fc_polar_workspace_bytes(ctypes.byref(L.PolarDesc(512, 2048, 8, 5, 1)), ctypes.byref(n16)) == 0
    # X, Y: 512 x 2048; A, B: 512 x 512; per matrix; bf16 halves the buffers
    assert n32.value >= 8 * 4 * (2 * 512 * 2048 + 2 * 512 * 512)
    assert n16.value < 0.51 * n32.value + 8 * 1024
    assert L.lib().fc_polar_workspace_bytes(ctypes.byref(L.PolarDesc(0, 4, 1, 5, 0)), ctypes.byref(n32)) == 1
    assert L.lib().fc_polar_workspace_bytes(ctypes.byref(L.PolarDesc(4, 4, 1, 5, 7)), ctypes.byref(n32)) == 1
