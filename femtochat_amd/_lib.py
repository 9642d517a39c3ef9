"""ctypes binding of libfemtochat_attn.so (the C ABI in include/femtochat_attn.h
include/femtochat_loss.h, include/femtochat_optim.h and include/femtochat_xla.h).

The shared library is built in-tree by ``femtochat_amd.build`` (hipcc,
gfx950).  Loading fails loudly when it is missing: there is no CPU fallback
behind this module.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_NAME = "libfemtochat_attn.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

FC_OK = 0
FC_ERR_INVALID_ARGUMENT = 1
FC_ERR_UNSUPPORTED = 2
FC_ERR_WORKSPACE = 3
FC_ERR_HIP = 4

FC_F32 = 0
FC_BF16 = 1
FC_MODE_EXACT = 0
FC_MODE_FAST = 1
FC_FLAG_OVERWRITE = 1
FC_PASS_FORWARD = 0
FC_PASS_BACKWARD = 1
FC_REDUCE_NONE = 0
FC_REDUCE_SUM = 1
FC_REDUCE_MEAN = 2
FC_INDEX_I32 = 0
FC_INDEX_I64 = 1

STATUS_NAMES = {
    FC_OK: "FC_OK",
    FC_ERR_INVALID_ARGUMENT: "FC_ERR_INVALID_ARGUMENT",
    FC_ERR_UNSUPPORTED: "FC_ERR_UNSUPPORTED",
    FC_ERR_WORKSPACE: "FC_ERR_WORKSPACE",
    FC_ERR_HIP: "FC_ERR_HIP",
}


class AttnDesc(ctypes.Structure):
    _fields_ = [
        ("D", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("Hkv", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("B", ctypes.c_int32),
        ("win_left", ctypes.c_int32),
        ("win_right", ctypes.c_int32),
        ("mode", ctypes.c_int32),
        ("in_dtype", ctypes.c_int32),
        ("out_dtype", ctypes.c_int32),
        ("dout_dtype", ctypes.c_int32),
        ("grad_dtype", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
    ]


class RopeNormDesc(ctypes.Structure):
    _fields_ = [
        ("D", ctypes.c_int32),
        ("NH", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("B", ctypes.c_int32),
        ("table_len", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
    ]


class XentDesc(ctypes.Structure):
    _fields_ = [
        ("V", ctypes.c_int32),
        ("index_base", ctypes.c_int32),
        ("N", ctypes.c_int64),
        ("ignore_index", ctypes.c_int64),
        ("index_type", ctypes.c_int32),
        ("reduction", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
    ]


class EmbedDesc(ctypes.Structure):
    _fields_ = [
        ("D", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("N", ctypes.c_int64),
        ("index_base", ctypes.c_int32),
        ("index_type", ctypes.c_int32),
        ("y_dtype", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
    ]


class AdamWDesc(ctypes.Structure):
    _fields_ = [
        ("n", ctypes.c_int64),
        ("t", ctypes.c_int32),
        ("alpha", ctypes.c_float),
        ("beta1", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("lam", ctypes.c_float),
        ("grad_scale", ctypes.c_float),
    ]


class PolarDesc(ctypes.Structure):
    _fields_ = [
        ("m", ctypes.c_int32),
        ("n", ctypes.c_int32),
        ("count", ctypes.c_int32),
        ("steps", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
    ]


class Caps(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 64),
        ("arch", ctypes.c_char * 32),
        ("compute_units", ctypes.c_int32),
        ("wavefront_size", ctypes.c_int32),
        ("lds_bytes_per_block", ctypes.c_int32),
        ("max_threads_per_block", ctypes.c_int32),
        ("clock_khz", ctypes.c_int32),
        ("global_mem_bytes", ctypes.c_int64),
    ]


class KernelTime(ctypes.Structure):
    _fields_ = [
        ("kernel", ctypes.c_char * 48),
        ("launches", ctypes.c_int32),
        ("total_ms", ctypes.c_double),
    ]


# The callback type of an XLA FFI call site: bool callback(void* stream, void** buffers).
XLA_CALLBACK = ctypes.CFUNCTYPE(ctypes.c_bool, ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p))


class AttentionError(RuntimeError):
    """A non-zero fc_status from the library, with its message."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


_lib = None

_P = ctypes.c_void_p
_SIGNATURES = {
    "fc_abi_version": (ctypes.c_int32, []),
    "fc_last_error": (ctypes.c_char_p, []),
    "fc_attn_supported_head_dims": (ctypes.c_uint32, []),
    "fc_attn_workspace_bytes": (
        ctypes.c_int,
        [ctypes.POINTER(AttnDesc), ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(ctypes.c_size_t)],
    ),
    "fc_attn_fwd": (
        ctypes.c_int,
        [ctypes.POINTER(AttnDesc), _P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _P],
    ),
    "fc_attn_bwd": (
        ctypes.c_int,
        [ctypes.POINTER(AttnDesc), _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _P],
    ),
    "fc_attn_bwd_noalloc": (
        ctypes.c_int,
        [ctypes.POINTER(AttnDesc), _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    ),
    "fc_rope_norm_fwd": (ctypes.c_int, [ctypes.POINTER(RopeNormDesc), _P, _P, _P, _P, _P, _P]),
    "fc_rope_norm_bwd": (ctypes.c_int, [ctypes.POINTER(RopeNormDesc), _P, _P, _P, _P, _P, _P, _P]),
    "fc_cross_entropy_fwd": (ctypes.c_int, [ctypes.POINTER(XentDesc), _P, _P, _P, _P, _P, _P, _P]),
    "fc_cross_entropy_count": (ctypes.c_int, [ctypes.POINTER(XentDesc), _P, _P, _P]),
    "fc_cross_entropy_bwd": (ctypes.c_int, [ctypes.POINTER(XentDesc), _P, _P, _P, _P, _P, _P, _P]),
    "fc_cross_entropy_fused": (ctypes.c_int, [ctypes.POINTER(XentDesc), _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "fc_embedding_fwd": (ctypes.c_int, [ctypes.POINTER(EmbedDesc), _P, _P, _P, _P]),
    "fc_embedding_bwd": (ctypes.c_int, [ctypes.POINTER(EmbedDesc), _P, _P, _P, _P]),
    "fc_embedding_bwd_workspace_bytes": (ctypes.c_int, [ctypes.POINTER(EmbedDesc), ctypes.POINTER(ctypes.c_size_t)]),
    "fc_embedding_bwd_sorted": (ctypes.c_int, [ctypes.POINTER(EmbedDesc), _P, _P, _P, _P, ctypes.c_size_t, _P]),
    "fc_xla_bind_attention_fwd": (ctypes.c_void_p, [ctypes.POINTER(AttnDesc), ctypes.c_int32]),
    "fc_xla_bind_attention_bwd": (ctypes.c_void_p, [ctypes.POINTER(AttnDesc), ctypes.c_int32,
                                                    ctypes.POINTER(ctypes.c_size_t)]),
    "fc_xla_bind_embedding_fwd": (ctypes.c_void_p, [ctypes.POINTER(EmbedDesc)]),
    "fc_xla_bind_embedding_bwd": (ctypes.c_void_p, [ctypes.POINTER(EmbedDesc)]),
    "fc_xla_last_error": (ctypes.c_char_p, []),
    "fc_adamw_step": (ctypes.c_int, [ctypes.POINTER(AdamWDesc), _P, _P, _P, _P, _P]),
    "fc_adam_update": (ctypes.c_int, [ctypes.c_int64, ctypes.c_int64, ctypes.c_float, ctypes.c_float,
                                      _P, _P, _P, _P, _P, _P, _P]),
    "fc_muon_update": (ctypes.c_int, [ctypes.c_int64, ctypes.c_int32, _P, _P, _P, _P, _P, _P]),
    "fc_param_gather": (ctypes.c_int, [ctypes.c_int64, ctypes.c_int32, _P, _P, _P, _P]),
    "fc_param_scatter": (ctypes.c_int, [ctypes.c_int64, ctypes.c_int32, _P, _P, _P, _P]),
    "fc_polar_workspace_bytes": (ctypes.c_int, [ctypes.POINTER(PolarDesc), ctypes.POINTER(ctypes.c_size_t)]),
    "fc_polar_express": (ctypes.c_int, [ctypes.POINTER(PolarDesc), _P, _P, ctypes.c_size_t, _P]),
    "fc_polar_express_grouped": (ctypes.c_int, [ctypes.c_int32, ctypes.POINTER(PolarDesc), ctypes.POINTER(_P),
                                                ctypes.POINTER(_P), ctypes.POINTER(ctypes.c_size_t), _P]),
    "fc_convert": (ctypes.c_int, [_P, ctypes.c_int32, _P, ctypes.c_int32, ctypes.c_int64, _P]),
    "fc_fill_zero": (ctypes.c_int, [_P, ctypes.c_size_t, _P]),
    "fc_capabilities": (ctypes.c_int, [ctypes.c_int32, ctypes.POINTER(Caps)]),
    "fc_profile_enable": (ctypes.c_int, [ctypes.c_int32]),
    "fc_profile_collect": (
        ctypes.c_int,
        [ctypes.POINTER(KernelTime), ctypes.c_int32, ctypes.POINTER(ctypes.c_int32)],
    ),
}


def lib():
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        path = Path(os.environ.get("FEMTOCHAT_ATTN_LIB", LIB_PATH))
        if not path.exists():
            raise RuntimeError(
                f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "(hipcc, gfx950). There is no CPU fallback."
            )
        handle = ctypes.CDLL(str(path))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != FC_OK:
        msg = lib().fc_last_error().decode(errors="replace")
        raise AttentionError(status, msg)


def profile_enable(on: bool) -> None:
    check(lib().fc_profile_enable(1 if on else 0))


def profile_collect() -> dict:
    """{kernel name: (launches, total_ms)} since the last collection."""
    cap = 64
    buf = (KernelTime * cap)()
    n = ctypes.c_int32(0)
    check(lib().fc_profile_collect(buf, cap, ctypes.byref(n)))
    return {
        buf[i].kernel.decode(): (int(buf[i].launches), float(buf[i].total_ms)) for i in range(min(n.value, cap))
    }
