"""femtochat's optimizer kernels on the MI355X.

====================================================  ==========================================================
reference (Julia)                                     here (Python, torch tensors on a HIP device)
====================================================  ==========================================================
``AdamW(θ; α, β₁, β₂, ϵ, λ, t)``, ``ω(θ, g; Nₜ)``     ``AdamW(theta, alpha=, beta1=, ...)``, ``opt(theta, g, grad_scale=)``
(src/optim.jl:11-94)
``adam_update_kernel!`` (CUDAExt:99-106)              ``adam_update_(Theta, offset, m, v, alpha, beta, eta, lam, eps)``
``muon_update_kernel!`` (CUDAExt:108-119)             ``muon_update_(Theta, X, eta, lam, offsets)``
``gather!`` / ``scatter!`` (src/optim.jl:262-276)      ``gather_(stack, vector, offsets)`` / ``scatter_(vector, stack, offsets)``
``polar_express!(G, work, steps)`` (:129-149)         ``polar_express_(G, steps=5, workspace=None)``, ``polar_express``
====================================================  ==========================================================

Arrays are float32.  Matrices follow the reference's column-major storage:
a Julia (m, n, k) stack is a torch (k, n, m) tensor (each [j] is G[:, :, j]
transposed in torch's row-major view); ``polar_express_`` takes that
(k, n, m) tensor and the Julia sizes are read from it.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib
from .kernels import _ptr, _stream_ptr

__all__ = ["AdamW", "adamw_step_", "adam_update_", "muon_update_", "gather_", "scatter_", "polar_express_",
           "polar_express_grouped_", "polar_express", "polar_workspace_bytes"]


def _f32(name, t, device=None):
    if not isinstance(t, torch.Tensor) or t.dtype != torch.float32 or not t.is_contiguous():
        raise TypeError(f"{name} must be a contiguous float32 tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: the MI355X optimizer kernels need tensors on a HIP device; there is no CPU path")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")


def adamw_step_(theta, grad, m, v, t: int, alpha, beta1, beta2, eps, lam, grad_scale=1.0) -> None:
    """One AdamW step in place (moments, decay, bias-corrected update) at step count t."""
    for name, x in (("theta", theta), ("grad", grad), ("m", m), ("v", v)):
        _f32(name, x, theta.device)
        if x.numel() != theta.numel():
            raise ValueError(f"{name} has {x.numel()} elements, theta {theta.numel()}")
    d = _lib.AdamWDesc(theta.numel(), int(t), alpha, beta1, beta2, eps, lam, grad_scale)
    _lib.check(_lib.lib().fc_adamw_step(ctypes.byref(d), _ptr(theta), _ptr(grad), _ptr(m), _ptr(v),
                                        _stream_ptr(theta.device)))


class AdamW:
    """The reference's ``AdamW`` state (zero moments, step count t) with its
    call ``ω(θ, g; α, Nₜ)`` as one fused kernel.  Hyperparameters are float32,
    as ``MuonAdamW`` constructs them."""

    def __init__(self, theta: torch.Tensor, alpha=0.001, beta1=0.9, beta2=0.999, eps=1e-8, lam=0.01, t: int = 0):
        _f32("theta", theta)
        self.alpha, self.beta1, self.beta2, self.eps, self.lam, self.t = alpha, beta1, beta2, eps, lam, t
        self.m = torch.zeros_like(theta)
        self.v = torch.zeros_like(theta)

    def __call__(self, theta: torch.Tensor, grad: torch.Tensor, alpha=None, grad_scale=1.0) -> None:
        self.t += 1
        adamw_step_(theta, grad, self.m, self.v, self.t, self.alpha if alpha is None else alpha, self.beta1,
                    self.beta2, self.eps, self.lam, grad_scale)


def adam_update_(Theta, offset: int, m, v, alpha, beta, eta, lam: float, eps: float) -> None:
    """Theta[offset:offset+n] = Theta (1 - eta lam) - alpha m / (sqrt(v / beta) + eps); alpha, beta
    and eta are 1-element device tensors."""
    for name, x in (("Theta", Theta), ("m", m), ("v", v), ("alpha", alpha), ("beta", beta), ("eta", eta)):
        _f32(name, x, Theta.device)
    if offset < 0 or offset + m.numel() > Theta.numel() or v.numel() != m.numel():
        raise ValueError("m, v and Theta[offset:offset+len(m)] must match")
    _lib.check(_lib.lib().fc_adam_update(m.numel(), offset, lam, eps, _ptr(Theta), _ptr(m), _ptr(v), _ptr(alpha),
                                         _ptr(beta), _ptr(eta), _stream_ptr(Theta.device)))


def _offsets(offsets, width, vector, count, validate=True):
    """Checks the offsets tensor; with ``validate`` also its values (which
    reads them back from the device: a caller that builds its offsets once, as
    the reference's ``muon_group`` does, checks them once and then passes
    ``validate=False``)."""
    if offsets.dtype != torch.int64 or offsets.device != vector.device or offsets.numel() != count:
        raise TypeError("offsets must be a device int64 tensor with one entry per matrix")
    if validate:
        lo, hi = int(offsets.min()), int(offsets.max())
        if lo < 0 or hi + width > vector.numel():
            raise ValueError("an offset puts a matrix outside the flat storage")


def muon_update_(Theta, X, eta, lam, offsets, *, validate: bool = True) -> None:
    """Cautious Muon write of the stacked X (count, width) into the flat Theta."""
    for name, x in (("Theta", Theta), ("X", X), ("eta", eta), ("lam", lam)):
        _f32(name, x, Theta.device)
    count, width = X.shape[0], X[0].numel()
    _offsets(offsets, width, Theta, count, validate)
    _lib.check(_lib.lib().fc_muon_update(width, count, _ptr(Theta), _ptr(X), _ptr(eta), _ptr(lam), _ptr(offsets),
                                         _stream_ptr(Theta.device)))


def gather_(stack, vector, offsets, *, validate: bool = True) -> None:
    _f32("stack", stack, vector.device)
    _f32("vector", vector)
    count, width = stack.shape[0], stack[0].numel()
    _offsets(offsets, width, vector, count, validate)
    _lib.check(_lib.lib().fc_param_gather(width, count, _ptr(stack), _ptr(vector), _ptr(offsets),
                                          _stream_ptr(vector.device)))


def scatter_(vector, stack, offsets, *, validate: bool = True) -> None:
    _f32("stack", stack, vector.device)
    _f32("vector", vector)
    count, width = stack.shape[0], stack[0].numel()
    _offsets(offsets, width, vector, count, validate)
    _lib.check(_lib.lib().fc_param_scatter(width, count, _ptr(vector), _ptr(stack), _ptr(offsets),
                                           _stream_ptr(vector.device)))


def _polar_desc(G, steps, compute_type=torch.float32):
    if G.dim() != 3:
        raise ValueError("G must be a (k, n, m) stack (the Julia (m, n, k) array)")
    if compute_type not in (torch.float32, torch.bfloat16):
        raise ValueError("compute_type must be torch.float32 or torch.bfloat16")
    k, n, m = G.shape
    return _lib.PolarDesc(m, n, k, int(steps), _lib.FC_BF16 if compute_type == torch.bfloat16 else _lib.FC_F32)


def polar_workspace_bytes(G: torch.Tensor, steps: int = 5, compute_type=torch.float32) -> int:
    n = ctypes.c_size_t(0)
    _lib.check(_lib.lib().fc_polar_workspace_bytes(ctypes.byref(_polar_desc(G, steps, compute_type)),
                                                   ctypes.byref(n)))
    return n.value


def polar_express_(G: torch.Tensor, steps: int = 5, workspace: Optional[torch.Tensor] = None,
                   compute_type=torch.float32) -> torch.Tensor:
    """Polar Express in place on the stack G (see the module docstring for the
    layout); ``compute_type=torch.bfloat16`` runs the iteration in bf16 as the
    reference's ``compute_type=BFloat16`` workspace does."""
    _f32("G", G)
    d = _polar_desc(G, steps, compute_type)
    nbytes = polar_workspace_bytes(G, steps, compute_type)
    if workspace is None:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=G.device)
    if workspace.numel() < nbytes or workspace.device != G.device:
        raise ValueError(f"the workspace must hold {nbytes} bytes on {G.device}")
    _lib.check(_lib.lib().fc_polar_express(ctypes.byref(d), _ptr(G), _ptr(workspace), workspace.numel(),
                                           _stream_ptr(G.device)))
    return G


def polar_express_grouped_(stacks, steps: int = 5, workspaces=None, compute_type=torch.float32):
    """Polar Express in place on several stacks at once (the reference's Muon
    groups, one per matrix shape), run concurrently on helper streams forked
    from and joined to the current stream."""
    stacks = list(stacks)
    if not stacks:
        return stacks
    dev = stacks[0].device
    for G in stacks:
        _f32("G", G, dev)
    descs = (_lib.PolarDesc * len(stacks))(*[_polar_desc(G, steps, compute_type) for G in stacks])
    sizes = [polar_workspace_bytes(G, steps, compute_type) for G in stacks]
    if workspaces is None:
        workspaces = [torch.empty(n, dtype=torch.uint8, device=dev) for n in sizes]
    for w, n in zip(workspaces, sizes):
        if w.numel() < n or w.device != dev:
            raise ValueError("each workspace must hold polar_workspace_bytes(G) bytes on G's device")
    gp = (ctypes.c_void_p * len(stacks))(*[G.data_ptr() for G in stacks])
    wp = (ctypes.c_void_p * len(stacks))(*[w.data_ptr() for w in workspaces])
    wb = (ctypes.c_size_t * len(stacks))(*[w.numel() for w in workspaces])
    _lib.check(_lib.lib().fc_polar_express_grouped(len(stacks), descs, gp, wp, wb, _stream_ptr(dev)))
    return stacks


def polar_express(G: torch.Tensor, steps: int = 5, compute_type=torch.float32) -> torch.Tensor:
    return polar_express_(G.clone(), steps, compute_type=compute_type)
