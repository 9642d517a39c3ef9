"""The five attention workloads the library is measured and checked on, and
their synthetic inputs.

C1..C5 follow the benchmark contract of this project: the reference's README
toy model (README.md:46-85), a d12-scale layer in exact mode, the d20-scale
GQA layer (the headline workload), an 'SSSL' sliding-window stack, and packed
documents at long context.  Windows come from ``window_sizes``
(src/parameters.jl:200-210); positions restart at 0 at each document start as
the reference's loader produces them (src/dataloader.jl:157-174,241-274).

Inputs are generated on the host with numpy's PCG64 from a fixed seed per
(config, layer, tensor), so every run and every checker sees the same bytes.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Tuple

import numpy as np

from .kernels import window_sizes


@dataclass(frozen=True)
class Workload:
    name: str
    D: int
    H: int
    Hkv: int
    T: int
    B: int
    mode: str  # "exact" (fp32) or "fast" (bf16)
    windows: Tuple[Tuple[int, int], ...]
    rms_qk: bool = True
    dO_std: float = 0.1
    positions: str = "none"  # "none" | "linear" | "toy" | "documents"
    doc_mean: int = 400
    doc_sigma: float = 1.0
    doc_cap: int = 4096
    description: str = ""

    @property
    def layers(self) -> int:
        return len(self.windows)


def _c4_windows():
    return tuple(window_sizes(2048, 4, "SSSL"))


WORKLOADS = {
    "C1": Workload("C1", D=16, H=2, Hkv=1, T=4, B=2, mode="exact", windows=tuple(window_sizes(4, 1, "L")),
                   rms_qk=False, dO_std=1.0, positions="toy",
                   description="README toy GPT attention: n_embed=32, n_head=2, n_kv_head=1, T=4, B=2, fp32"),
    "C2": Workload("C2", D=128, H=6, Hkv=6, T=2048, B=8, mode="exact", windows=tuple(window_sizes(2048, 1, "L")),
                   positions="linear", description="d12-scale layer, fp32 exact, full causal"),
    "C3": Workload("C3", D=128, H=10, Hkv=5, T=2048, B=16, mode="fast", windows=tuple(window_sizes(2048, 1, "L")),
                   description="d20-scale GQA 2:1, bf16, full causal (headline workload)"),
    "C4": Workload("C4", D=128, H=10, Hkv=10, T=2048, B=16, mode="fast", windows=_c4_windows(),
                   description="'SSSL' sliding windows over 4 layers, bf16"),
    "C5": Workload("C5", D=128, H=16, Hkv=8, T=8192, B=4, mode="fast", windows=tuple(window_sizes(8192, 1, "L")),
                   positions="documents",
                   description="packed documents (lognormal lengths, mean 400, cap 4096), T=8192, bf16"),
}


def _seed(workload: Workload, layer: int, tensor: int) -> int:
    return 1000 * int(workload.name[1:]) + 100 * layer + tensor


def _normal(seed: int, shape, std: float = 1.0) -> np.ndarray:
    x = np.random.Generator(np.random.PCG64(seed)).standard_normal(shape, dtype=np.float32)
    if std != 1.0:
        x *= np.float32(std)
    return x


def _unit_rms(x: np.ndarray) -> np.ndarray:
    return x / np.sqrt(np.mean(np.square(x, dtype=np.float64), axis=-1, keepdims=True)).astype(np.float32)


def document_positions(T: int, B: int, seed: int, mean: int = 400, sigma: float = 1.0, cap: int = 4096,
                       mid_document_start: bool = True) -> np.ndarray:
    """(B, T) int32 positions for rows packed with documents whose lengths are
    lognormal with the given mean (mu = ln(mean) - sigma^2/2), capped at
    ``cap``; positions restart at 0 per document.  The first document of a
    row may start part-way through (positions beginning above 0), as a
    loader continuing a long document does (src/dataloader.jl:258)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    mu = np.log(mean) - sigma * sigma / 2.0
    out = np.zeros((B, T), np.int32)
    for b in range(B):
        t = 0
        first = True
        while t < T:
            n = int(min(cap, max(1, round(float(rng.lognormal(mu, sigma))))))
            start = int(rng.integers(0, n)) if (first and mid_document_start) else 0
            first = False
            take = min(n - start, T - t)
            out[b, t:t + take] = np.arange(start, start + take, dtype=np.int32)
            t += take
    return out


def positions_for(workload: Workload, layer: int = 0) -> Optional[np.ndarray]:
    T, B = workload.T, workload.B
    if workload.positions == "none":
        return None
    if workload.positions == "linear":
        return np.tile(np.arange(T, dtype=np.int32), (B, 1))
    if workload.positions == "toy":
        # Int32[0:3 8:11] (README.md:63): column b of the (T,B) Julia matrix.
        return np.stack([np.arange(T, dtype=np.int32) + 8 * b for b in range(B)])
    if workload.positions == "documents":
        return document_positions(T, B, _seed(workload, layer, 5), workload.doc_mean, workload.doc_sigma,
                                  workload.doc_cap)
    raise ValueError(workload.positions)


@dataclass
class HostInputs:
    """float32 host arrays (already rounded to bf16 values in fast mode)."""

    Q: np.ndarray
    K: np.ndarray
    V: np.ndarray
    dO: np.ndarray
    positions: Optional[np.ndarray]
    window: Tuple[int, int]
    extra: dict = field(default_factory=dict)


def _round_bf16(x: np.ndarray) -> np.ndarray:
    import torch

    return torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()


def host_inputs(workload: Workload, layer: int = 0, batch: Optional[List[int]] = None) -> HostInputs:
    """Synthetic inputs of one layer.  ``batch`` selects rows (the values of a
    row do not depend on which rows are selected)."""
    B = workload.B
    rows = list(range(B)) if batch is None else list(batch)
    T, H, Hkv, D = workload.T, workload.H, workload.Hkv, workload.D

    def gen(tensor, heads, std=1.0, rms=False):
        parts = []
        for b in rows:
            x = _normal(_seed(workload, layer, tensor) * 10007 + b, (T, heads, D), std)
            parts.append(_unit_rms(x) if rms else x)
        return np.stack(parts)

    Q = gen(1, H, rms=workload.rms_qk)
    K = gen(2, Hkv, rms=workload.rms_qk)
    V = gen(3, Hkv)
    dO = gen(4, H, std=workload.dO_std)
    if workload.mode == "fast":
        Q, K, V, dO = (_round_bf16(x) for x in (Q, K, V, dO))
    pos = positions_for(workload, layer)
    if pos is not None:
        pos = pos[rows]
    return HostInputs(Q, K, V, dO, pos, tuple(workload.windows[layer]))


def device_inputs(workload: Workload, layer: int = 0, device="cuda", batch=None):
    """(Q, K, V, dO, positions) torch tensors on ``device`` in the workload's dtype."""
    import torch

    h = host_inputs(workload, layer, batch)
    dt = torch.bfloat16 if workload.mode == "fast" else torch.float32
    t = [torch.from_numpy(x).to(device=device, dtype=dt).contiguous() for x in (h.Q, h.K, h.V, h.dO)]
    pos = None if h.positions is None else torch.from_numpy(h.positions).to(device=device).contiguous()
    return t[0], t[1], t[2], t[3], pos, h.window


def visible_pairs(T: int, B: int, H: int, window, positions: Optional[np.ndarray] = None) -> int:
    """Visible (query, key) pairs summed over rows and heads, counted from the
    per-query key interval [lb, ub] (no T x T mask is built)."""
    left, right = int(window[0]), int(window[1])
    q = np.arange(T, dtype=np.int64)
    if (left, right) == (-1, 0):
        lb, ub = np.zeros(T, np.int64), q.copy()
    else:
        lb, ub = q - left, q + right
    lb = np.maximum(lb, 0)
    ub = np.minimum(ub, T - 1)
    total = 0
    for b in range(B):
        lbb = lb if positions is None else np.maximum(lb, q - positions[b].astype(np.int64))
        total += int(np.maximum(ub - lbb + 1, 0).sum())
    return total * H


def flops(workload: Workload) -> dict:
    """Algorithmic FLOPs over all layers (visible pairs only): fwd 4*D per pair,
    bwd 10*D per pair (the FlashAttention convention)."""
    pairs = 0
    for layer in range(workload.layers):
        pairs += visible_pairs(workload.T, workload.B, workload.H, workload.windows[layer],
                               positions_for(workload, layer))
    D = workload.D
    return {"pairs": pairs, "fwd": 4 * D * pairs, "bwd": 10 * D * pairs, "total": 14 * D * pairs}
