"""Host-side logic (CPU only): window generation, workloads, pair counting,
document positions, and the Python mirror's argument checking."""
import numpy as np
import pytest
import torch

from femtochat_amd import MFMAExact, MFMAFast, accumulator_type, attention_, attention_inputs, window_sizes
from femtochat_amd import kernels as Kn
from femtochat_amd import workloads as W
from oracle import attention_ref as R


def test_window_sizes_reference_semantics():
    # src/parameters.jl:200-210: S = min(L, cld(L,512)*128), last layer forced to L.
    assert window_sizes(2048, 4, "SSSL") == [(512, 0), (512, 0), (512, 0), (2048, 0)]
    assert window_sizes(4, 2, "L") == [(4, 0), (4, 0)]
    assert window_sizes(2048, 3, "S") == [(512, 0), (512, 0), (2048, 0)]
    assert window_sizes(1000, 2, "SL") == [(256, 0), (1000, 0)]
    assert window_sizes(100, 1, "S") == [(100, 0)]
    # The reference tests `== 'S'` only: every other character is a long layer.
    assert window_sizes(2048, 4, "SXsL") == [(512, 0), (2048, 0), (2048, 0), (2048, 0)]
    assert window_sizes(2048, 3, "x") == [(2048, 0)] * 3
    assert window_sizes(2048, 5, "SL") == [(512, 0), (2048, 0), (512, 0), (2048, 0), (2048, 0)]
    # mod1(i, 0) and windows[end] on an empty list fail in the reference too.
    with pytest.raises(ValueError):
        window_sizes(2048, 2, "")
    with pytest.raises(ValueError):
        window_sizes(2048, 0, "S")


def test_visible_pairs_matches_mask_count():
    for T, window in ((37, (-1, 0)), (50, (7, 0)), (64, (5, 3)), (20, (0, 0)), (30, (-1, 4))):
        pos = W.document_positions(T, 2, seed=T, mean=8, sigma=1.0, cap=30)
        for p in (None, pos):
            assert W.visible_pairs(T, 2, 3, window, p) == R.visible_pairs(T, 2, 3, window, p)


def test_workload_flops_match_baseline_table():
    f = W.flops(W.WORKLOADS["C3"])
    assert f["pairs"] == 335_708_160 and f["total"] == 14 * 128 * 335_708_160
    assert W.flops(W.WORKLOADS["C2"])["pairs"] == 100_712_448
    assert W.flops(W.WORKLOADS["C4"])["pairs"] == 776_970_240
    assert W.flops(W.WORKLOADS["C1"])["pairs"] == 40


def test_document_positions_properties():
    pos = W.document_positions(8192, 4, seed=5, mean=400, sigma=1.0, cap=4096)
    assert pos.shape == (4, 8192) and pos.dtype == np.int32
    for row in pos:
        starts = np.flatnonzero(np.diff(row) != 1) + 1
        assert np.all(row[starts] == 0)              # a new document restarts at 0
        assert row.max() < 4096                       # capped length
        seg = np.split(row, starts)
        assert all(np.all(np.diff(s) == 1) for s in seg)
    lengths = np.diff(np.flatnonzero(np.concatenate([pos[0] == 0, [True]])))
    assert 150 < lengths.mean() < 900


def test_host_inputs_deterministic_and_normalised():
    wl = W.WORKLOADS["C3"]
    a = W.host_inputs(wl, batch=[3])
    b = W.host_inputs(wl, batch=[3])
    assert np.array_equal(a.Q, b.Q) and np.array_equal(a.dO, b.dO)
    rms = np.sqrt((a.Q.astype(np.float64) ** 2).mean(-1))
    assert np.allclose(rms, 1.0, atol=1e-2)  # unit RMS before bf16 rounding
    assert np.array_equal(a.Q, torch.from_numpy(a.Q).bfloat16().float().numpy())  # bf16-representable
    assert abs(a.dO.std() - 0.1) < 0.01


def test_instruction_contract():
    assert accumulator_type(MFMAFast(), torch.bfloat16) == torch.float32
    assert accumulator_type(MFMAExact(), torch.float32) == torch.float32
    q = torch.zeros(1, 4, 2, 16)
    qc, kc, vc = attention_inputs(MFMAFast(), q, q, q)
    assert qc.dtype == torch.bfloat16
    qc, _, _ = attention_inputs(MFMAExact(), q.bfloat16(), q, q)
    assert qc.dtype == torch.float32


def test_python_mirror_rejects_bad_arguments_before_the_library():
    Q = torch.zeros(1, 8, 4, 16, dtype=torch.bfloat16)
    K = torch.zeros(1, 8, 2, 16, dtype=torch.bfloat16)
    O = torch.zeros_like(Q)
    l = torch.zeros(1, 4, 8)
    with pytest.raises(ValueError, match="HIP device"):
        attention_(MFMAFast(), O, l, l.clone(), Q, K, K, (-1, 0))
    with pytest.raises(ValueError, match="shape"):
        attention_(MFMAFast(), O, l, l.clone(), Q, K[:, :4], K, (-1, 0))
    with pytest.raises(ValueError, match="multiple"):
        attention_(MFMAFast(), O, l, l.clone(), Q, K[:, :, :1].expand(1, 8, 3, 16).contiguous(), K, (-1, 0))
    with pytest.raises(TypeError, match="dtype"):
        attention_(MFMAExact(), O, l, l.clone(), Q, K, K, (-1, 0))
    with pytest.raises(TypeError, match="MFMAExact"):
        attention_(object(), O, l, l.clone(), Q, K, K, (-1, 0))
    with pytest.raises(TypeError, match="unexpected keyword"):
        attention_(MFMAFast(), O, l, l.clone(), Q, K, K, (-1, 0), bogus=1)


def test_geometry_keywords_are_accepted():
    # scripts/train.jl:26 passes backward=(; warps=Val(4), query_tile=Val(64)).
    Kn._reject_unknown({"warps": 4, "query_tile": 64, "head_span": 1})


def test_build_flags_keep_ieee_nan_and_packed_fp32_off():
    # Every HIP source builds with IEEE NaN semantics (a NaN query must reach
    # its own row's outputs, as Julia's max and exp carry it) and with packed
    # FP32 instructions disabled for the device code.
    from femtochat_amd import build as B
    flags = list(B.HIPCC_FLAGS) + [f for extra in B.EXTRA_FLAGS.values() for f in extra]
    for bad in ("-ffast-math", "-fno-honor-nans", "-ffinite-math-only", "-funsafe-math-optimizations"):
        assert bad not in flags, bad
    seq = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
    assert any(flags[i:i + 4] == seq for i in range(len(flags) - 3))
