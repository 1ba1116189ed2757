"""Fused RMSNorm and residual-add + RMSNorm on gfx950 (libumic_hip.so).

Drop-in for the reference's ``rmsnorm_triton`` / ``add_rmsnorm_triton``
(src/umic/kernels/rmsnorm.py:53-73 and :103-134): same arguments, same
[..., N] in / out shapes, outputs allocated by torch on the current stream.
One launch per call; each element of x (and the residual) is read once and
each output written once.

Numerics follow the eager HF ``Qwen3VLTextRMSNorm`` chain the kernel replaces
(transformers modeling_qwen3_vl.py:400-405): fp32 normalisation rounded to
bf16, then the bf16 weight multiply rounded again.  ``add_rmsnorm`` adds the
residual as the eager decoder layer does -- one bf16 rounding, and the norm
is taken of that rounded sum, which is also the returned residual stream.
"""

from __future__ import annotations

import torch

from umic import _lib
from umic.kernels._common import ld, require_device, rows2d, vec


def rmsnorm_eligible(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """True if the HIP kernel reproduces the eager module on these inputs."""
    return (x.is_cuda and x.dtype == torch.bfloat16 and isinstance(weight, torch.Tensor)
            and weight.dtype == torch.bfloat16 and weight.dim() == 1
            and weight.device == x.device and x.dim() >= 1
            and x.shape[-1] == weight.shape[0] and x.shape[-1] > 0)


def rmsnorm_hip(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the last dim: bf16(w * bf16(x * rsqrt(mean(x^2) + eps)))."""
    require_device(x, weight)
    shape = x.shape
    x2d = rows2d(x)
    M, N = x2d.shape
    out = torch.empty((M, N), dtype=x.dtype, device=x.device)
    w = vec(weight)
    with _lib.device_of(x):
        _lib.call("umic_rmsnorm_bf16", x2d.data_ptr(), w.data_ptr(), out.data_ptr(),
                  M, N, ld(x2d), N, float(eps), _lib.stream_of(x))
    return out.reshape(shape)


def add_rmsnorm_hip(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                    eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Return (rmsnorm(bf16(x + residual)) * w, bf16(x + residual))."""
    require_device(x, residual, weight)
    if residual.shape != x.shape:
        raise ValueError(f"residual shape {tuple(residual.shape)} != x shape {tuple(x.shape)}")
    shape = x.shape
    x2d, r2d = rows2d(x), rows2d(residual)
    M, N = x2d.shape
    normed = torch.empty((M, N), dtype=x.dtype, device=x.device)
    summed = torch.empty((M, N), dtype=x.dtype, device=x.device)
    w = vec(weight)
    with _lib.device_of(x):
        _lib.call("umic_add_rmsnorm_bf16", x2d.data_ptr(), r2d.data_ptr(), w.data_ptr(),
                  normed.data_ptr(), summed.data_ptr(), M, N, ld(x2d), ld(r2d), N, N,
                  float(eps), _lib.stream_of(x))
    return normed.reshape(shape), summed.reshape(shape)


def _last_pow2(v: int) -> int:
    p = 1
    while p * 2 <= v:
        p *= 2
    return p


# Rows and LDS limit of the decode launches that fold the norm into a GEMV
# (umic_rmsnorm_linear_multi_bf16, umic_add_rmsnorm_gate_silu_mul_bf16).
GEMV_NORM_MAX_ROWS = 2
GEMV_NORM_MAX_LDS = 64 << 10


def wide_plan(rows: int, n: int) -> tuple[int, int] | None:
    """(bw, k4) of torch's RMSNorm reduction plan (Reduce.cuh's
    setReduceConfig for a contiguous fp32 [rows, n] reduced over n, as the
    library's ``rms_plan`` restates it) when the library runs it as its wide
    single-block kernel -- 4-vectors, no row split, bw >= 128 reducing
    threads with k4 <= 8 vectors each -- else None.  The GEMV-folded norms
    reproduce exactly this plan."""
    if rows < 1 or n < 128 or n % 4:
        return None
    dim0 = n // 4
    d0 = _last_pow2(dim0) if dim0 < 512 else 512
    d1 = _last_pow2(rows) if rows < 512 else 512
    bw = d0 if d0 < 64 else 64
    bh = d1 if d1 < 512 // bw else 512 // bw
    bw = d0 if d0 < 512 // bh else 512 // bh
    vpt = -(-n // bw)
    if vpt >= min(bh * 16, 256) or bw < 128:
        return None
    k4 = -(-(n // 4) // bw)
    return (bw, k4) if k4 <= 8 else None


# 4-vectors per thread and row the folded norm holds in registers (its 256
# threads play bw reducing threads with k4 vectors each).
GEMV_NORM_MAX_PV = 4


def gemv_norm_ok(rows: int, n: int) -> bool:
    """True if a decode GEMV over rows x n can fold the RMSNorm of its input."""
    if not (1 <= rows <= GEMV_NORM_MAX_ROWS and n % 8 == 0 and rows * n * 2 <= GEMV_NORM_MAX_LDS):
        return False
    plan = wide_plan(rows, n)
    return plan is not None and (2 if plan[0] > 256 else 1) * plan[1] <= GEMV_NORM_MAX_PV


# Names of the reference's wrappers (src/umic/kernels/rmsnorm.py:53, :103),
# kept so code written against that API runs unchanged on this runtime.
rmsnorm_triton = rmsnorm_hip
add_rmsnorm_triton = add_rmsnorm_hip
