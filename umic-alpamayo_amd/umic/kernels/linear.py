"""bf16 linear (x @ W^T [+ bias] [+ erf-GELU]) on gfx950 MFMA (libumic_hip.so).

Drop-in for the reference's ``linear_triton`` (src/umic/kernels/linear.py:
118-145): the weight is the nn.Linear [N, K] tensor, read in place (the MFMA
kernel consumes K-contiguous rows of both operands, so there is no transpose
and no copy).  fp32 accumulation, bias and GELU applied to the fp32
accumulator, one bf16 rounding.  Site selection (which Linear modules use it)
lives in umic.integrate, as in the reference.
"""

from __future__ import annotations

import ctypes

import torch

from umic import _lib
from umic.kernels._common import ld, require_device, rows2d

K_MULTIPLE = 32  # the kernel's K step
N_MULTIPLE = 8   # 16-byte output runs


def _gemm_ready(t2d: torch.Tensor) -> torch.Tensor:
    """Row-major view with a 16-byte aligned base and row stride (else a copy)."""
    if t2d.stride(-1) != 1 or (t2d.shape[0] > 1 and t2d.stride(0) % 8) or t2d.data_ptr() % 16:
        t2d = t2d.contiguous()
    return t2d


def linear_eligible(x: torch.Tensor, weight: torch.Tensor, bias=None) -> bool:
    """True if (x, weight, bias) can run on the HIP kernel."""
    if not (x.is_cuda and x.dtype == torch.bfloat16 and isinstance(weight, torch.Tensor)
            and weight.dtype == torch.bfloat16 and weight.dim() == 2
            and weight.device == x.device and x.dim() >= 1):
        return False
    N, K = weight.shape
    if x.shape[-1] != K or K % K_MULTIPLE or N % N_MULTIPLE or K == 0:
        return False
    if bias is not None and not (bias.dtype == torch.bfloat16 and bias.dim() == 1
                                 and bias.shape[0] == N and bias.device == x.device):
        return False
    return True


_ACT_CODES = {None: _lib.UMIC_ACT_NONE, "gelu": _lib.UMIC_ACT_GELU,
              "gelu_tanh": _lib.UMIC_ACT_GELU_TANH}


def linear_hip(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
               act: str | None = None) -> torch.Tensor:
    """Compute act(x @ weight.T + bias).

    Args:
        x: [..., K] activations, bf16 on the GPU.
        weight: [N, K] nn.Linear weight (read in place).
        bias: optional [N].
        act: None, "gelu" (erf GELU epilogue) or "gelu_tanh" (tanh-approximate
            GELU, torch's gelu(approximate="tanh")).
    """
    require_device(x, weight, *([bias] if bias is not None else []))
    if act not in _ACT_CODES:
        raise ValueError(f"unsupported activation {act!r}")
    if not linear_eligible(x, weight, bias):
        raise ValueError(f"linear_hip: unsupported shape x{tuple(x.shape)} w{tuple(weight.shape)}"
                         f" (need K % {K_MULTIPLE} == 0 and N % {N_MULTIPLE} == 0)")
    shape = x.shape
    x2d = _gemm_ready(rows2d(x))
    w = _gemm_ready(weight)
    b = None if bias is None else bias.contiguous()
    M, K = x2d.shape
    N = w.shape[0]
    out = torch.empty((M, N), dtype=x.dtype, device=x.device)
    with _lib.device_of(x):
        stream = _lib.stream_of(x)
        ws, ws_bytes = workspace(x.device, stream, M, N, K)
        _lib.call("umic_linear_ws_bf16", x2d.data_ptr(), w.data_ptr(), _lib.ptr(b), out.data_ptr(),
                  M, N, K, ld(x2d), ld(w), N,
                  _ACT_CODES[act],
                  _lib.ptr(ws), ws_bytes, stream)
    return out.reshape(*shape[:-1], N)


GEMV_MAX_ROWS = 8  # rows the decode GEMV (and umic_linear_multi_bf16) takes


def linear_multi_hip(x: torch.Tensor, weights, biases=None) -> list[torch.Tensor]:
    """[x @ w.T + b for each (w, b)] in one launch (umic_linear_multi_bf16):
    the decode GEMV over up to three linears that share x, e.g. the
    attention's q/k/v projections.  x has 1..GEMV_MAX_ROWS rows; every pair
    must pass ``linear_eligible``.  Each result equals ``linear_hip`` on its
    linear bit for bit (same kernel)."""
    biases = list(biases) if biases is not None else [None] * len(weights)
    require_device(x, *weights, *[b for b in biases if b is not None])
    if not 1 <= len(weights) <= 3 or len(biases) != len(weights):
        raise ValueError("linear_multi_hip: one to three linears")
    x2d = _gemm_ready(rows2d(x))
    M, K = x2d.shape
    if not 1 <= M <= GEMV_MAX_ROWS:
        raise ValueError(f"linear_multi_hip: {M} rows (decode GEMV takes 1..{GEMV_MAX_ROWS})")
    for w, b in zip(weights, biases):
        if not linear_eligible(x, w, b):
            raise ValueError(f"linear_multi_hip: unsupported shape x{tuple(x.shape)} "
                             f"w{tuple(w.shape)}")
    ws = [_gemm_ready(w) for w in weights]
    bs = [None if b is None else b.contiguous() for b in biases]
    outs = [torch.empty((M, w.shape[0]), dtype=x.dtype, device=x.device) for w in ws]
    n = len(ws)
    P, I64 = ctypes.c_void_p * n, ctypes.c_int64 * n
    with _lib.device_of(x):
        _lib.call("umic_linear_multi_bf16", x2d.data_ptr(), M, K, ld(x2d), n,
                  P(*[w.data_ptr() for w in ws]), P(*[_lib.ptr(b) for b in bs]),
                  P(*[o.data_ptr() for o in outs]), I64(*[w.shape[0] for w in ws]),
                  I64(*[ld(w) for w in ws]), I64(*[w.shape[0] for w in ws]), 0,
                  _lib.stream_of(x))
    return [o.reshape(*x.shape[:-1], o.shape[1]) for o in outs]


def rmsnorm_linear_multi_hip(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, weights,
                             biases=None) -> list[torch.Tensor]:
    """[rmsnorm(x) @ w.T + b for each (w, b)] in one launch
    (umic_rmsnorm_linear_multi_bf16): the decode step's input RMSNorm folded
    into the q/k/v GEMV, bit-identical to ``rmsnorm_hip`` then
    ``linear_multi_hip``.  x has 1..GEMV_NORM_MAX_ROWS rows whose norm plan
    ``rmsnorm.gemv_norm_ok`` accepts."""
    from umic.kernels import rmsnorm

    biases = list(biases) if biases is not None else [None] * len(weights)
    require_device(x, norm_weight, *weights, *[b for b in biases if b is not None])
    if not 1 <= len(weights) <= 3 or len(biases) != len(weights):
        raise ValueError("rmsnorm_linear_multi_hip: one to three linears")
    x2d = _gemm_ready(rows2d(x))
    M, K = x2d.shape
    if not rmsnorm.gemv_norm_ok(M, K) or tuple(norm_weight.shape) != (K,):
        raise ValueError(f"rmsnorm_linear_multi_hip: {M} x {K} rows are not a foldable norm")
    for w, b in zip(weights, biases):
        if not linear_eligible(x, w, b):
            raise ValueError(f"rmsnorm_linear_multi_hip: unsupported shape x{tuple(x.shape)} "
                             f"w{tuple(w.shape)}")
    nw = norm_weight.contiguous()
    ws = [_gemm_ready(w) for w in weights]
    bs = [None if b is None else b.contiguous() for b in biases]
    outs = [torch.empty((M, w.shape[0]), dtype=x.dtype, device=x.device) for w in ws]
    n = len(ws)
    P, I64 = ctypes.c_void_p * n, ctypes.c_int64 * n
    with _lib.device_of(x):
        _lib.call("umic_rmsnorm_linear_multi_bf16", x2d.data_ptr(), nw.data_ptr(), None, M, K,
                  ld(x2d), K, float(eps), n,
                  P(*[w.data_ptr() for w in ws]), P(*[_lib.ptr(b) for b in bs]),
                  P(*[o.data_ptr() for o in outs]), I64(*[w.shape[0] for w in ws]),
                  I64(*[ld(w) for w in ws]), I64(*[w.shape[0] for w in ws]),
                  _lib.stream_of(x))
    return [o.reshape(*x.shape[:-1], o.shape[1]) for o in outs]


def linear_add_hip(x: torch.Tensor, weight: torch.Tensor, bias, residual: torch.Tensor):
    """residual + (x @ weight.T + bias), rounded as the eager chain rounds
    (the linear's bf16 output, then the bf16 sum), in one decode-GEMV launch
    (umic_linear_add_bf16).  x has 1..GEMV_MAX_ROWS rows; residual has the
    output's shape."""
    require_device(x, weight, residual, *([bias] if bias is not None else []))
    if not linear_eligible(x, weight, bias):
        raise ValueError(f"linear_add_hip: unsupported shape x{tuple(x.shape)} "
                         f"w{tuple(weight.shape)}")
    x2d = _gemm_ready(rows2d(x))
    M, K = x2d.shape
    N = weight.shape[0]
    if not 1 <= M <= GEMV_MAX_ROWS:
        raise ValueError(f"linear_add_hip: {M} rows (decode GEMV takes 1..{GEMV_MAX_ROWS})")
    if residual.shape != (*x.shape[:-1], N) or residual.dtype != x.dtype:
        raise ValueError(f"linear_add_hip: residual {tuple(residual.shape)} does not match "
                         f"the output {(*x.shape[:-1], N)}")
    w = _gemm_ready(weight)
    b = None if bias is None else bias.contiguous()
    r2d = rows2d(residual.contiguous())
    out = torch.empty((M, N), dtype=x.dtype, device=x.device)
    with _lib.device_of(x):
        _lib.call("umic_linear_add_bf16", x2d.data_ptr(), w.data_ptr(), _lib.ptr(b),
                  r2d.data_ptr(), out.data_ptr(), M, N, K, ld(x2d), ld(w), N, N,
                  _lib.stream_of(x))
    return out.reshape(*x.shape[:-1], N)


def stream_k_planned(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """True if linear_hip(x, weight) runs the stream-K schedule on this device."""
    if not x.is_cuda:
        return False
    M = x.numel() // x.shape[-1] if x.shape[-1] else 0
    N, K = weight.shape
    with _lib.device_of(x):
        return _lib.lib().umic_linear_workspace_bytes(M, N, K) > 0


# Stream-K workspaces, one per (device, stream): the kernel leaves its
# counters at zero after every launch, so a workspace is zeroed once, when it
# is created, and reused by every later call on that stream (calls on one
# stream never overlap).
_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}
# Workspaces replaced by a larger one stay allocated: a HIP graph captured
# earlier still holds the old address, and its replays must not write into
# memory the caching allocator has handed to another tensor.  Growth at
# least doubles, so few are ever retired.
_RETIRED: list[torch.Tensor] = []


def workspace(device: torch.device, stream: int, M: int, N: int, K: int):
    """(tensor, bytes) the stream-K linear needs for this shape, or (None, 0).

    One zeroed workspace per (device, stream): the kernel leaves its counters
    at zero after every call, and calls on one stream never overlap."""
    need = _lib.lib().umic_linear_workspace_bytes(M, N, K)
    if need <= 0:
        return None, 0
    key = (device.index, stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < need:
        if ws is not None:
            _RETIRED.append(ws)
            need = max(need, 2 * ws.numel())
        ws = torch.zeros(need, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws, ws.numel()


# Name of the reference's wrapper (src/umic/kernels/linear.py:118).
linear_triton = linear_hip
