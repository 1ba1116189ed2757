"""Fused LayerNorm and residual-add + LayerNorm on gfx950 (libumic_hip.so).

Drop-in for the reference's ``layernorm_triton`` / ``add_layernorm_triton``
(src/umic/kernels/layernorm.py:54-68 and :102-124).  Last-dim LayerNorm with
affine weight and bias, biased variance, fp32 statistics and one bf16
rounding of ``w * (rstd * (x - mean)) + b`` -- the numerics of
``torch.nn.functional.layer_norm`` on bf16 tensors.  ``add_layernorm`` adds
the residual with one bf16 rounding first (the eager ViT block's
``hidden_states + attn(...)``) and normalises that rounded sum.
"""

from __future__ import annotations

import torch

from umic import _lib
from umic.kernels._common import ld, require_device, rows2d, vec


def layernorm_eligible(x: torch.Tensor, weight, bias) -> bool:
    return (x.is_cuda and x.dtype == torch.bfloat16
            and isinstance(weight, torch.Tensor) and isinstance(bias, torch.Tensor)
            and weight.dtype == torch.bfloat16 and bias.dtype == torch.bfloat16
            and weight.dim() == 1 and bias.dim() == 1
            and weight.device == x.device and bias.device == x.device
            and x.dim() >= 1 and x.shape[-1] == weight.shape[0] == bias.shape[0]
            and x.shape[-1] > 0)


def layernorm_hip(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                  eps: float) -> torch.Tensor:
    """LayerNorm over the last dim; fp32 statistics, bf16 output."""
    require_device(x, weight, bias)
    shape = x.shape
    x2d = rows2d(x)
    M, N = x2d.shape
    out = torch.empty((M, N), dtype=x.dtype, device=x.device)
    w, b = vec(weight), vec(bias)
    with _lib.device_of(x):
        _lib.call("umic_layernorm_bf16", x2d.data_ptr(), w.data_ptr(), b.data_ptr(),
                  out.data_ptr(), M, N, ld(x2d), N, float(eps), _lib.stream_of(x))
    return out.reshape(shape)


def add_layernorm_hip(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                      bias: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Return (layernorm(bf16(x + residual)), bf16(x + residual))."""
    require_device(x, residual, weight, bias)
    if residual.shape != x.shape:
        raise ValueError(f"residual shape {tuple(residual.shape)} != x shape {tuple(x.shape)}")
    shape = x.shape
    x2d, r2d = rows2d(x), rows2d(residual)
    M, N = x2d.shape
    normed = torch.empty((M, N), dtype=x.dtype, device=x.device)
    summed = torch.empty((M, N), dtype=x.dtype, device=x.device)
    w, b = vec(weight), vec(bias)
    with _lib.device_of(x):
        _lib.call("umic_add_layernorm_bf16", x2d.data_ptr(), r2d.data_ptr(), w.data_ptr(),
                  b.data_ptr(), normed.data_ptr(), summed.data_ptr(), M, N, ld(x2d), ld(r2d),
                  N, N, float(eps), _lib.stream_of(x))
    return normed.reshape(shape), summed.reshape(shape)


# Names of the reference's wrappers (src/umic/kernels/layernorm.py:54, :102).
layernorm_triton = layernorm_hip
add_layernorm_triton = add_layernorm_hip
