"""femtochat's attention plug-in API, served by the MI355X (gfx950) library.

This module mirrors the reference's attention interface so that a caller of
``FemtoChat.Kernels`` finds the same entry points with the same meaning:

====================================  =============================================
reference (Julia)                     here (Python, torch tensors on a HIP device)
====================================  =============================================
``attention(Q, K, V, window)``        ``attention(Q, K, V, window)``
``attention(𝒜, Q, K, V, window)``     ``attention(MFMAFast(), Q, K, V, window)``
``attention!(𝒜, O, ℓ, m, Q, K, V, w)`` ``attention_(𝒜, O, l, m, Q, K, V, w)``
``Δattention!(𝒜, dQ, dK, dV, dO, …)``  ``delta_attention_(𝒜, dQ, dK, dV, dO, …)``
``attention_state(𝒜, Q, K, V, w)``    ``attention_state(𝒜, Q, K, V, w)``
``accumulator_type(𝒜, F)``            ``accumulator_type(𝒜, dtype)``
``attention_inputs(𝒜, Q, K, V)``      ``attention_inputs(𝒜, Q, K, V)``
``SIMTInstruction`` / ``TensorCore…``  ``MFMAExact`` / ``MFMAFast``
``window_sizes(config)``              ``window_sizes(sequence_len, n_layer, pattern)``
====================================  =============================================

References: src/kernels.jl:417-433 (API), ext/FemtoChatCUDAExt.jl:210-241
(instruction selection, conversions), ext/FemtoChatCUDAExt.jl:1242-1260 and
:1747-1790 (keyword contract: unknown launch-geometry keywords are accepted,
``accumulate`` selects add versus overwrite), src/parameters.jl:200-210
(window_sizes).

Layout: a Julia array of size (D,H,T,B) (column-major) is the same memory as a
torch tensor of shape (B,T,H,D) (row-major); the statistics ℓ and m, (1,T,H,B)
in Julia, are torch tensors of shape (B,H,T).  positions, (T,B) Int32 in
Julia, is a (B,T) int32 tensor.  ``window`` is the reference's (left, right)
tuple with (-1, 0) meaning causal.

New relative to the reference: ``positions=`` enables a document mask (key k
is visible to query q only if k >= q - positions[q]); ``positions=None`` is the
reference's behaviour exactly.
"""
from __future__ import annotations

import ctypes
from typing import NamedTuple, Optional, Tuple

import torch

from . import _lib

__all__ = [
    "MFMAExact",
    "MFMAFast",
    "attention",
    "attention_",
    "delta_attention_",
    "backward_workspace_bytes",
    "forward_workspace_bytes",
    "attention_state",
    "accumulator_type",
    "attention_inputs",
    "instruction",
    "window_sizes",
    "capabilities",
    "AttentionFunction",
    "AttentionState",
]

# Keywords of the reference's CUDA launchers (ext/FemtoChatCUDAExt.jl:1246,1775)
# that select CUDA launch geometry.  They are accepted and ignored so that a
# reference `attention_options` NamedTuple (scripts/train.jl:26) still works.
_GEOMETRY_KEYWORDS = {"warps", "query_tile", "head_span", "order", "query_subtiles", "key_tile", "simt"}


class MFMAExact:
    """fp32 inputs, fp32 MFMA, fp32 outputs: the analogue of the reference's
    ``SIMTInstruction`` (ext/FemtoChatCUDAExt.jl:210, kernels :243-1002)."""

    mode = _lib.FC_MODE_EXACT

    def __repr__(self) -> str:
        return "MFMAExact()"

    def __eq__(self, other) -> bool:
        return type(other) is type(self)

    def __hash__(self) -> int:
        return hash(type(self))


class MFMAFast:
    """bf16 Q/K/V with bf16 MFMA and fp32 accumulation/statistics: the analogue of
    ``TensorCoreInstruction`` (ext/FemtoChatCUDAExt.jl:211, kernels :1004-2068)."""

    mode = _lib.FC_MODE_FAST

    def __repr__(self) -> str:
        return "MFMAFast()"

    def __eq__(self, other) -> bool:
        return type(other) is type(self)

    def __hash__(self) -> int:
        return hash(type(self))


Instruction = (MFMAExact, MFMAFast)


class AttentionState(NamedTuple):
    """The saved forward state ``(; 𝒜, Q, K, V, O, ℓ, m)`` (src/kernels.jl:425-433)."""

    A: object
    Q: torch.Tensor
    K: torch.Tensor
    V: torch.Tensor
    O: torch.Tensor
    l: torch.Tensor
    m: torch.Tensor


def window_sizes(sequence_len: int, n_layer: int, window_pattern: str = "L"):
    """Per-layer ``(left, 0)`` windows: 'S' -> ``(min(L, cld(L, 512)*128), 0)``,
    any other character -> ``(L, 0)``, last layer forced to ``(L, 0)``
    (src/parameters.jl:200-210, which tests ``== 'S'`` only).  An empty
    pattern or no layers is an error there too (``mod1(i, 0)``, ``windows[end]``)."""
    if n_layer <= 0:
        raise ValueError("n_layer must be positive")
    if not window_pattern:
        raise ValueError("window_pattern must not be empty")
    L = int(sequence_len)
    S = min(L, -(-L // 512) * 128)
    windows = [(S, 0) if window_pattern[i % len(window_pattern)] == "S" else (L, 0) for i in range(n_layer)]
    windows[-1] = (L, 0)
    return windows


def _dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return _lib.FC_F32
    if dtype == torch.bfloat16:
        return _lib.FC_BF16
    raise TypeError(f"unsupported dtype {dtype}; the library stores float32 or bfloat16")


def instruction(dtype: torch.dtype, device=None, D: Optional[int] = None):
    """Default implementation for a dtype and head dim, like the reference's
    ``instruction(F, dev, Val(D))`` (ext/FemtoChatCUDAExt.jl:214-223): the
    matrix-core path (fast) for float32/bfloat16/float16 when ``0 < D <= 128``
    and ``D % 16 == 0``.  Shapes the library cannot run raise instead of
    falling back to a CPU path."""
    if dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise TypeError(f"no HIP attention for dtype {dtype}")
    if D is not None:
        mask = _lib.lib().fc_attn_supported_head_dims()
        if not (0 < D <= 128 and D % 16 == 0 and (mask >> (D // 16 - 1)) & 1):
            raise _lib.AttentionError(_lib.FC_ERR_UNSUPPORTED, f"head_dim {D} is not supported")
    return MFMAFast()


def accumulator_type(A, dtype: torch.dtype) -> torch.dtype:
    """Statistics are float32 for both instructions (ext/FemtoChatCUDAExt.jl:228)."""
    if isinstance(A, Instruction):
        return torch.float32
    return dtype


def convert_(dst: torch.Tensor, src: torch.Tensor) -> None:
    """dst := src converted by the library (``fc_convert``): float32 and
    bfloat16 in either direction, round to nearest even; both contiguous on
    one GPU with the same number of elements."""
    for name, t in (("dst", dst), ("src", src)):
        if t.dtype not in (torch.float32, torch.bfloat16) or not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 or bfloat16 GPU tensor")
    if dst.numel() != src.numel() or dst.device != src.device:
        raise ValueError("dst and src must have the same number of elements on the same device")
    _lib.check(_lib.lib().fc_convert(_ptr(src), _dtype_code(src.dtype), _ptr(dst), _dtype_code(dst.dtype),
                                     src.numel(), _stream_ptr(src.device)))


def fill_zero_(t: torch.Tensor) -> torch.Tensor:
    """t := 0 by the library's fill kernel (``fc_fill_zero``)."""
    if not t.is_cuda or not t.is_contiguous():
        raise ValueError("fill_zero_ needs a contiguous GPU tensor")
    _lib.check(_lib.lib().fc_fill_zero(_ptr(t), t.numel() * t.element_size(), _stream_ptr(t.device)))
    return t


def attention_inputs(A, Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor):
    """Precision conversion before the forward (ext/FemtoChatCUDAExt.jl:229-230):
    the fast path stores Q/K/V in bfloat16, the exact path in float32.  GPU
    tensors are converted by the library (``fc_convert``)."""
    if isinstance(A, MFMAFast):
        target = torch.bfloat16
    elif isinstance(A, MFMAExact):
        target = torch.float32
    else:
        return Q, K, V

    def conv(x):
        if x.dtype == target:
            return x
        if x.is_cuda and x.dtype in (torch.float32, torch.bfloat16):
            y = torch.empty(x.shape, dtype=target, device=x.device)
            convert_(y, x.contiguous())
            return y
        return x.to(target)

    return tuple(conv(x) for x in (Q, K, V))


def _stream_ptr(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _check_tensor(name, t, shape, dtypes, device):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if t.dtype not in dtypes:
        raise TypeError(f"{name} has dtype {t.dtype}, expected one of {dtypes}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _stats_shape(t: torch.Tensor, B: int, H: int, T: int):
    return (B, H, T, 1) if t.dim() == 4 else (B, H, T)


def _desc(A, Q, K, window, out_dtype, dout_dtype, grad_dtype, overwrite=False) -> _lib.AttnDesc:
    if not isinstance(A, Instruction):
        raise TypeError(f"expected MFMAExact() or MFMAFast(), got {A!r}")
    if Q.dim() != 4 or K.dim() != 4:
        raise ValueError("Q, K, V must be 4-d (B, T, H, D) tensors")
    B, T, H, D = Q.shape
    Hkv = K.shape[2]
    left, right = (int(window[0]), int(window[1]))
    d = _lib.AttnDesc()
    d.D, d.H, d.Hkv, d.T, d.B = D, H, Hkv, T, B
    d.win_left, d.win_right = left, right
    d.mode = A.mode
    d.in_dtype = _dtype_code(Q.dtype)
    d.out_dtype = out_dtype
    d.dout_dtype = dout_dtype
    d.grad_dtype = grad_dtype
    d.flags = _lib.FC_FLAG_OVERWRITE if overwrite else 0
    return d


def _check_common(A, Q, K, V, positions):
    device = Q.device
    if not isinstance(A, Instruction):
        raise TypeError(f"expected MFMAExact() or MFMAFast(), got {A!r}")
    if Q.dim() != 4:
        raise ValueError("Q must have shape (B, T, H, D)")
    B, T, H, D = Q.shape
    in_dtypes = (torch.bfloat16,) if isinstance(A, MFMAFast) else (torch.float32,)
    _check_tensor("Q", Q, (B, T, H, D), in_dtypes, device)
    if K.dim() != 4:
        raise ValueError("K must have shape (B, T, Hkv, D)")
    Hkv = K.shape[2]
    if Hkv <= 0 or H % Hkv != 0:
        raise ValueError(f"n_head {H} is not a multiple of n_kv_head {Hkv}")
    _check_tensor("K", K, (B, T, Hkv, D), in_dtypes, device)
    _check_tensor("V", V, (B, T, Hkv, D), in_dtypes, device)
    if positions is not None:
        _check_tensor("positions", positions, (B, T), (torch.int32,), device)
    if device.type != "cuda":
        raise ValueError("the MI355X attention path needs tensors on a HIP device (torch 'cuda'); there is no CPU path")
    return device, B, T, H, Hkv, D


def attention_(A, O, l, m, Q, K, V, window: Tuple[int, int], *, positions=None,
               workspace: Optional[torch.Tensor] = None, **options) -> None:
    """Forward into caller buffers: ``attention!(𝒜, O, ℓ, m, Q, K, V, window)``
    (src/kernels.jl:419; ext/FemtoChatCUDAExt.jl:1242-1260).  O is bfloat16 or
    float32 (fast) / float32 (exact); ℓ and m are float32 (B,H,T).  With
    positions in fast mode the library orders the query tiles by their work
    in a small workspace (allocated here unless ``workspace`` is given, of
    ``forward_workspace_bytes`` bytes); other problems need none."""
    _reject_unknown(options)
    device, B, T, H, Hkv, D = _check_common(A, Q, K, V, positions)
    out_dtypes = (torch.bfloat16, torch.float32) if isinstance(A, MFMAFast) else (torch.float32,)
    _check_tensor("O", O, (B, T, H, D), out_dtypes, device)
    _check_tensor("l", l, _stats_shape(l, B, H, T), (torch.float32,), device)
    _check_tensor("m", m, _stats_shape(m, B, H, T), (torch.float32,), device)
    oc = _dtype_code(O.dtype)
    d = _desc(A, Q, K, window, oc, oc, oc)
    lib = _lib.lib()
    nbytes = ctypes.c_size_t(0)
    _lib.check(lib.fc_attn_workspace_bytes(ctypes.byref(d), _lib.FC_PASS_FORWARD, int(positions is not None),
                                           ctypes.byref(nbytes)))
    ws, aligned = None, None
    if nbytes.value > 0:
        if workspace is None:
            ws = torch.empty(int(nbytes.value) + 256, dtype=torch.uint8, device=device)
        else:
            ws = workspace
            if ws.device != device or ws.numel() * ws.element_size() < int(nbytes.value) + 256:
                raise ValueError(f"workspace must be a {int(nbytes.value) + 256}-byte tensor on {device}")
        aligned = ctypes.c_void_p((ws.data_ptr() + 255) & ~255)
    _lib.check(
        lib.fc_attn_fwd(
            ctypes.byref(d), _ptr(Q), _ptr(K), _ptr(V), _ptr(positions), _ptr(O), _ptr(l), _ptr(m),
            aligned, ctypes.c_size_t(int(nbytes.value) if ws is not None else 0), _stream_ptr(device),
        )
    )


def delta_attention_(
    A, dQ, dK, dV, dO, Q, K, V, O, l, m, window: Tuple[int, int], *, positions=None, accumulate: bool = True,
    workspace: Optional[torch.Tensor] = None, **options,
) -> None:
    """Backward into caller buffers: ``Δattention!(𝒜, dQ, dK, dV, dO, Q, K, V, O,
    ℓ, m, window; accumulate=true)`` (src/kernels.jl:420;
    ext/FemtoChatCUDAExt.jl:1747-1790).  Adds into dQ/dK/dV unless
    ``accumulate=False``.  Gradients may be bfloat16 or float32 (fast mode)."""
    _reject_unknown(options)
    device, B, T, H, Hkv, D = _check_common(A, Q, K, V, positions)
    fast = isinstance(A, MFMAFast)
    io_dtypes = (torch.bfloat16, torch.float32) if fast else (torch.float32,)
    _check_tensor("dO", dO, (B, T, H, D), io_dtypes, device)
    _check_tensor("O", O, (B, T, H, D), io_dtypes, device)
    _check_tensor("l", l, _stats_shape(l, B, H, T), (torch.float32,), device)
    _check_tensor("m", m, _stats_shape(m, B, H, T), (torch.float32,), device)
    _check_tensor("dQ", dQ, (B, T, H, D), io_dtypes, device)
    _check_tensor("dK", dK, (B, T, Hkv, D), (dQ.dtype,), device)
    _check_tensor("dV", dV, (B, T, Hkv, D), (dQ.dtype,), device)
    d = _desc(A, Q, K, window, _dtype_code(O.dtype), _dtype_code(dO.dtype), _dtype_code(dQ.dtype),
              overwrite=not accumulate)
    lib = _lib.lib()
    nbytes = ctypes.c_size_t(0)
    _lib.check(lib.fc_attn_workspace_bytes(ctypes.byref(d), _lib.FC_PASS_BACKWARD, int(positions is not None),
                                           ctypes.byref(nbytes)))
    if workspace is None:
        ws = torch.empty(max(int(nbytes.value), 256) + 256, dtype=torch.uint8, device=device)
    else:
        ws = workspace
        if ws.device != device or ws.numel() * ws.element_size() < int(nbytes.value) + 256:
            raise ValueError(f"workspace must be a {int(nbytes.value) + 256}-byte tensor on {device}")
    base = ws.data_ptr()
    aligned = (base + 255) & ~255
    _lib.check(
        lib.fc_attn_bwd(
            ctypes.byref(d), _ptr(dO), _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(l), _ptr(m), _ptr(positions),
            _ptr(dQ), _ptr(dK), _ptr(dV), ctypes.c_void_p(aligned), ctypes.c_size_t(int(nbytes.value)),
            _stream_ptr(device),
        )
    )
    # An internally allocated workspace must outlive the kernels on this stream.
    if workspace is None:
        ws.record_stream(torch.cuda.current_stream(device))


def forward_workspace_bytes(A, Q, K, *, positions=None) -> int:
    """Bytes of the caller-owned workspace ``attention_(…, workspace=)``
    accepts (the library's requirement plus 256 bytes of alignment slack; 0
    when the problem needs none)."""
    d = _desc(A, Q, K, (-1, 0), _dtype_code(Q.dtype), _dtype_code(Q.dtype), _dtype_code(Q.dtype))
    n = ctypes.c_size_t(0)
    _lib.check(_lib.lib().fc_attn_workspace_bytes(ctypes.byref(d), _lib.FC_PASS_FORWARD,
                                                  int(positions is not None), ctypes.byref(n)))
    return int(n.value) + 256 if n.value > 0 else 0


def backward_workspace_bytes(A, Q, K, *, positions=None, dout_dtype=None) -> int:
    """Bytes of the caller-owned workspace ``delta_attention_(…, workspace=)``
    accepts (the library's requirement plus 256 bytes of alignment slack)."""
    dd = _dtype_code(dout_dtype or Q.dtype)
    d = _desc(A, Q, K, (-1, 0), dd, dd, dd)
    n = ctypes.c_size_t(0)
    _lib.check(_lib.lib().fc_attn_workspace_bytes(ctypes.byref(d), _lib.FC_PASS_BACKWARD,
                                                   int(positions is not None), ctypes.byref(n)))
    return int(n.value) + 256


def _reject_unknown(options: dict) -> None:
    unknown = set(options) - _GEOMETRY_KEYWORDS
    if unknown:
        raise TypeError(f"unexpected keyword(s) {sorted(unknown)}")


def attention_state(A, Q, K, V, window, *, positions=None, **options) -> AttentionState:
    """Allocate O, ℓ, m, convert inputs, run the forward and return the saved
    state (src/kernels.jl:425-433).  ``A`` may be the ``attention`` function
    itself, which selects the default instruction like
    ``attention_state(::typeof(attention), Q::CuArray, …)``
    (ext/FemtoChatCUDAExt.jl:225-226)."""
    if A is attention:
        A = instruction(Q.dtype, Q.device, Q.shape[-1])
    B, T, H, _ = Q.shape
    Qc, Kc, Vc = attention_inputs(A, Q, K, V)
    out_dtype = Q.dtype if Q.dtype in (torch.float32, torch.bfloat16) else torch.float32
    if isinstance(A, MFMAExact):
        out_dtype = torch.float32
    O = torch.empty(Q.shape, dtype=out_dtype, device=Q.device)
    F = accumulator_type(A, Q.dtype)
    l = torch.empty((B, H, T), dtype=F, device=Q.device)
    m = torch.empty((B, H, T), dtype=F, device=Q.device)
    attention_(A, O, l, m, Qc, Kc, Vc, window, positions=positions, **options)
    return AttentionState(A, Qc, Kc, Vc, O, l, m)


def attention(*args, positions=None, forward=None, backward=None, **options) -> torch.Tensor:
    """``attention(Q, K, V, window)`` or ``attention(𝒜, Q, K, V, window)``
    (src/kernels.jl:417; ext/FemtoChatCUDAExt.jl:235-241).  The
    ``forward=``/``backward=`` option channel of the reference's model call
    (src/gpt.jl:108) is accepted; only the forward options apply here."""
    opts = dict(forward or {})
    opts.update(options)
    if len(args) == 5:
        A, Q, K, V, window = args
    elif len(args) == 4:
        Q, K, V, window = args
        A = attention
    else:
        raise TypeError("attention(Q, K, V, window) or attention(A, Q, K, V, window)")
    return attention_state(A, Q, K, V, window, positions=positions, **opts).O


class AttentionFunction(torch.autograd.Function):
    """Differentiable attention, the role of the reference's Enzyme rule
    (ext/FemtoChatEnzymeExt.jl:221-278): forward = ``attention_state``; reverse =
    ``Δattention!`` accumulating into zero-initialised gradient buffers."""

    @staticmethod
    def forward(ctx, Q, K, V, window, A=None, positions=None):
        A = A if A is not None else instruction(Q.dtype, Q.device, Q.shape[-1])
        st = attention_state(A, Q, K, V, window, positions=positions)
        ctx.save_for_backward(st.Q, st.K, st.V, st.O, st.l, st.m, positions if positions is not None else Q.new_empty(0))
        ctx.A, ctx.window, ctx.has_pos = A, window, positions is not None
        ctx.dtypes = (Q.dtype, K.dtype, V.dtype)
        return st.O

    @staticmethod
    def backward(ctx, dO):
        Q, K, V, O, l, m, pos = ctx.saved_tensors
        positions = pos if ctx.has_pos else None
        gdtype = torch.float32
        dO = dO.contiguous()
        if dO.dtype != O.dtype:
            dO = dO.to(O.dtype)
        dQ = torch.zeros(Q.shape, dtype=gdtype, device=Q.device)
        dK = torch.zeros(K.shape, dtype=gdtype, device=Q.device)
        dV = torch.zeros(V.shape, dtype=gdtype, device=Q.device)
        delta_attention_(ctx.A, dQ, dK, dV, dO, Q, K, V, O, l, m, ctx.window, positions=positions)
        out = [g.to(dt) if g.dtype != dt else g for g, dt in zip((dQ, dK, dV), ctx.dtypes)]
        return out[0], out[1], out[2], None, None, None


def capabilities(device: int = 0) -> dict:
    """Device introspection, like the reference's ``capabilities()``
    (ext/FemtoChatCUDAExt.jl:177-208)."""
    caps = _lib.Caps()
    _lib.check(_lib.lib().fc_capabilities(int(device), ctypes.byref(caps)))
    return {
        "name": caps.name.decode(),
        "arch": caps.arch.decode(),
        "compute_units": caps.compute_units,
        "wavefront_size": caps.wavefront_size,
        "lds_bytes_per_block": caps.lds_bytes_per_block,
        "max_threads_per_block": caps.max_threads_per_block,
        "clock_khz": caps.clock_khz,
        "global_mem_bytes": caps.global_mem_bytes,
        "supported_head_dims": [16 * (i + 1) for i in range(8) if (_lib.lib().fc_attn_supported_head_dims() >> i) & 1],
    }
