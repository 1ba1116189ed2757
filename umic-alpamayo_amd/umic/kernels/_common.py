"""Shared checks for the kernel wrappers (device, dtype, 2-D row views)."""

from __future__ import annotations

import torch

from umic import _lib


def require_device(*tensors: torch.Tensor) -> None:
    """Raise unless every tensor is a bf16 GPU tensor and the library loaded.

    The wrappers are the fused path itself: they never fall back.  Routing
    ineligible inputs to the eager module is the injection layer's decision
    (umic.integrate), made before a wrapper is called.
    """
    for t in tensors:
        if not t.is_cuda:
            raise ValueError(f"umic kernels run on the GPU; got a tensor on {t.device}")
        if t.dtype != torch.bfloat16:
            raise TypeError(f"umic kernels take bfloat16 tensors; got {t.dtype}")
    dev = tensors[0].device
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    _lib.lib()  # raises UmicLibraryError if libumic_hip.so is unavailable


def grad_needed(*tensors) -> bool:
    """True when autograd would have to flow through a fused op: grad mode is
    on and some participating tensor requires grad.  The kernels have no
    backward, so such calls take the eager path and autograd records the
    same graph as without UMIC.  Under ``torch.no_grad()`` or
    ``torch.inference_mode()`` (the inference setting) this is one mode check.
    """
    if not torch.is_grad_enabled():
        return False
    return any(t is not None and t.requires_grad for t in tensors)


def rows2d(x: torch.Tensor) -> torch.Tensor:
    """[..., n] -> [rows, n] view with unit inner stride (copy only if needed)."""
    x2d = x.reshape(-1, x.shape[-1])
    if x2d.stride(-1) != 1:
        x2d = x2d.contiguous()
    return x2d


def ld(t2d: torch.Tensor) -> int:
    """Row stride of a 2-D view (a single row may report any stride)."""
    return t2d.stride(0) if t2d.shape[0] > 1 else t2d.shape[1]


def vec(w: torch.Tensor) -> torch.Tensor:
    return w if w.is_contiguous() else w.contiguous()
