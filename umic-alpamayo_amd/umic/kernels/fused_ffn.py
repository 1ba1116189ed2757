"""P5 gate_silu_mul: silu(x @ Wg) * (x @ Wu) in one gfx950 MFMA kernel.

Drop-in for the reference's src/umic/kernels/fused_ffn.py.  The eager chain
runs two GEMMs, SiLU and a multiply and round-trips three [M, N]
intermediates through HBM; here one kernel stages each x tile once for both
products, keeps the gate and up accumulators (fp32) side by side in
registers, applies silu(g) * u there and writes only the bf16 product.

Argument convention is the reference's: ``w_gate`` / ``w_up`` are [K, N],
normally the free ``.t()`` views of nn.Linear [N, K] weights, which the
kernel reads in place.  A genuinely row-major [K, N] matrix is transposed
once per call (a copy) -- supported, but not the fast path.
"""

from __future__ import annotations

import torch

from umic import _lib
from umic.kernels._common import ld, require_device, rows2d
from umic.kernels.linear import K_MULTIPLE, N_MULTIPLE, _gemm_ready


def gate_silu_mul_eager(x: torch.Tensor, w_gate: torch.Tensor,
                        w_up: torch.Tensor) -> torch.Tensor:
    """Eager reference (and the CPU path): silu(x @ w_gate) * (x @ w_up).

    Args:
        x: Activations [M, K].
        w_gate: Gate projection weight [K, N].
        w_up: Up projection weight [K, N].
    """
    return torch.nn.functional.silu(x @ w_gate) * (x @ w_up)


def _as_nk(w_kn: torch.Tensor) -> torch.Tensor:
    """[K, N] argument -> [N, K] rows with unit inner stride."""
    return _gemm_ready(w_kn.t())


def p5_eligible(x: torch.Tensor, w_gate_nk: torch.Tensor, w_up_nk: torch.Tensor) -> bool:
    """True if x and the two [N, K] weights can run on the fused kernel."""
    if not (x.is_cuda and x.dtype == torch.bfloat16 and x.dim() >= 1):
        return False
    for w in (w_gate_nk, w_up_nk):
        if not (isinstance(w, torch.Tensor) and w.dtype == torch.bfloat16 and w.dim() == 2
                and w.device == x.device):
            return False
    N, K = w_gate_nk.shape
    return (tuple(w_up_nk.shape) == (N, K) and x.shape[-1] == K and K > 0
            and K % K_MULTIPLE == 0 and N % N_MULTIPLE == 0)


def gate_silu_mul_hip(x: torch.Tensor, w_gate: torch.Tensor,
                      w_up: torch.Tensor) -> torch.Tensor:
    """Fused launch; x [..., K], w_gate / w_up [K, N] -> [..., N] bf16."""
    require_device(x, w_gate, w_up)
    wg, wu = _as_nk(w_gate), _as_nk(w_up)
    if not p5_eligible(x, wg, wu):
        raise ValueError(f"gate_silu_mul_hip: unsupported shape x{tuple(x.shape)} "
                         f"w{tuple(w_gate.shape)} (need K % {K_MULTIPLE} == 0, "
                         f"N % {N_MULTIPLE} == 0)")
    shape = x.shape
    x2d = _gemm_ready(rows2d(x))
    M, K = x2d.shape
    N = wg.shape[0]
    out = torch.empty((M, N), dtype=x.dtype, device=x.device)
    with _lib.device_of(x):
        _lib.call("umic_gate_silu_mul_bf16", x2d.data_ptr(), wg.data_ptr(), wu.data_ptr(),
                  out.data_ptr(), M, N, K, ld(x2d), ld(wg), ld(wu), N, _lib.stream_of(x))
    return out.reshape(*shape[:-1], N)


def add_rmsnorm_gate_silu_mul_hip(x: torch.Tensor, residual: torch.Tensor,
                                  norm_weight: torch.Tensor, eps: float, w_gate: torch.Tensor,
                                  w_up: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(gate_silu_mul(rmsnorm(bf16(x + residual))), bf16(x + residual)) in one
    launch (umic_add_rmsnorm_gate_silu_mul_bf16): the decode step's
    post-attention residual add and RMSNorm folded into the P5 GEMV,
    bit-identical to ``rmsnorm.add_rmsnorm_hip`` then ``gate_silu_mul_hip``.
    x and residual have 1..GEMV_NORM_MAX_ROWS rows that
    ``rmsnorm.gemv_norm_ok`` accepts; w_gate / w_up are [K, N] as for
    ``gate_silu_mul_hip``."""
    from umic.kernels import rmsnorm

    require_device(x, residual, norm_weight, w_gate, w_up)
    wg, wu = _as_nk(w_gate), _as_nk(w_up)
    if not p5_eligible(x, wg, wu):
        raise ValueError(f"add_rmsnorm_gate_silu_mul_hip: unsupported shape x{tuple(x.shape)} "
                         f"w{tuple(w_gate.shape)}")
    if residual.shape != x.shape or residual.dtype != x.dtype:
        raise ValueError(f"residual shape {tuple(residual.shape)} != x shape {tuple(x.shape)}")
    x2d, r2d = _gemm_ready(rows2d(x)), rows2d(residual).contiguous()
    M, K = x2d.shape
    if not rmsnorm.gemv_norm_ok(M, K) or tuple(norm_weight.shape) != (K,):
        raise ValueError(f"add_rmsnorm_gate_silu_mul_hip: {M} x {K} rows are not a foldable norm")
    N = wg.shape[0]
    nw = norm_weight.contiguous()
    out = torch.empty((M, N), dtype=x.dtype, device=x.device)
    summed = torch.empty((M, K), dtype=x.dtype, device=x.device)
    with _lib.device_of(x):
        _lib.call("umic_add_rmsnorm_gate_silu_mul_bf16", x2d.data_ptr(), r2d.data_ptr(),
                  nw.data_ptr(), None, summed.data_ptr(), wg.data_ptr(), wu.data_ptr(),
                  out.data_ptr(), M, N, K, ld(x2d), ld(r2d), K, K, ld(wg), ld(wu), N,
                  float(eps), _lib.stream_of(x))
    return out.reshape(*x.shape[:-1], N), summed.reshape(x.shape)


def gate_silu_mul(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """Best available implementation for the P5 motif (reference
    src/umic/kernels/fused_ffn.py:121-126): the HIP kernel for GPU tensors
    when libumic_hip.so loads, else the eager chain."""
    if x.is_cuda and _lib.available():
        return gate_silu_mul_hip(x, w_gate, w_up)
    return gate_silu_mul_eager(x, w_gate, w_up)


# Name of the reference's fused launcher (src/umic/kernels/fused_ffn.py:93).
gate_silu_mul_triton = gate_silu_mul_hip
