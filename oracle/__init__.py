"""CPU parity oracle for the UMIC hot path -- TEST INFRASTRUCTURE ONLY.

Numpy front end over ``lib/liboracle.so`` (built from ``umic_oracle.c`` by
``oracle/Makefile``).  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` import this package, and only as the
checker or the timed CPU baseline.  The product package (``umic``) never
imports it: a missing HIP library makes the product raise, it never routes
here.

Every function takes and returns numpy arrays; bf16 tensors are ``uint16``
arrays holding the raw bf16 bit patterns (``bf16_from_f32`` / ``f32_from_bf16``
convert with round-to-nearest-even).  The C file documents, per function, the
eager op chain it restates (transformers ``modeling_qwen3_vl.py`` line
numbers) and the reference kernel it stands in for.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "liboracle.so")

# gfx950 v_rcp_f32 / v_rsq_f32 as measured deltas from the correctly rounded
# values (tests/golden/make_gfx950_tables.py); kept alive for the C side.
HW_TABLES = os.path.join(os.path.dirname(_HERE), "tests", "golden", "gfx950_rcp_rsq.npz")
_tables: list[np.ndarray] = []

_lib = None


def build() -> None:
    """Compile liboracle.so with the committed Makefile (gcc)."""
    import subprocess

    subprocess.run(["make", "-s", "-B", "-C", _HERE, "lib/liboracle.so"], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run oracle.build())")
        lib = ctypes.CDLL(LIB_PATH)
        P, I64, F32, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int
        sig = {
            "orc_f32_to_bf16": [P, P, I64],
            "orc_bf16_to_f32": [P, P, I64],
            "orc_rmsnorm": [P, P, P, I64, I64, F32],
            "orc_rms_var": [P, P, I64, I64],
            "orc_add_rmsnorm": [P, P, P, P, P, I64, I64, F32],
            "orc_set_hw_tables": [P, I64, P],
            "orc_layernorm": [P, P, P, P, P, P, I64, I64, F32, I],
            "orc_add_layernorm": [P, P, P, P, P, P, I64, I64, F32, I],
            "orc_ln_scalar_stats": [P, P, P, I64, I64, F32, I],
            "orc_rope_text": [P, P, P, P, I64, I64, I64],
            "orc_rope_vision": [P, P, P, P, I64, I64, I64],
            "orc_gemm_nt_f32": [P, P, P, I64, I64, I64],
            "orc_gate_silu_mul": [P, P, P, P, I64, I64, I64, I],
            "orc_linear": [P, P, P, P, I64, I64, I64, I, I],
        }
        ret = {"orc_rmsnorm", "orc_rms_var", "orc_add_rmsnorm", "orc_layernorm",
               "orc_add_layernorm", "orc_ln_scalar_stats"}
        for name, args in sig.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int if name in ret else None
        with np.load(HW_TABLES, allow_pickle=False) as t:
            _tables[:] = [np.ascontiguousarray(t["rcp_delta"], np.int8),
                          np.ascontiguousarray(t["rsq_delta2"], np.uint8)]
        lib.orc_set_hw_tables(_tables[0].ctypes.data_as(ctypes.c_void_p), _tables[0].size,
                              _tables[1].ctypes.data_as(ctypes.c_void_p))
        _lib = lib
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what}: unsupported shape (code {rc})")


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _u16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype != np.uint16:
        raise TypeError(f"expected uint16 bf16 bits, got {a.dtype}")
    return a


def _f32(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def bf16_from_f32(a: np.ndarray) -> np.ndarray:
    """Round fp32 values to bf16 (RNE); returns uint16 bit patterns."""
    a = _f32(a)
    out = np.empty(a.shape, np.uint16)
    _load().orc_f32_to_bf16(_p(a), _p(out), a.size)
    return out


def f32_from_bf16(a: np.ndarray) -> np.ndarray:
    """Widen bf16 bit patterns to fp32 (exact)."""
    a = _u16(a)
    return (a.astype(np.uint32) << 16).view(np.float32)


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """HF Qwen3VLTextRMSNorm over the last dim, in torch-ROCm's reduction
    order for a [rows, n] input (rows = every leading dim)."""
    x, w = _u16(x), _u16(w)
    n = x.shape[-1]
    y = np.empty_like(x)
    _check(_load().orc_rmsnorm(_p(x), _p(w), _p(y), x.size // n, n, eps), "rmsnorm")
    return y


def rms_var(x: np.ndarray) -> np.ndarray:
    """torch-ROCm's fp32 x.float().pow(2).mean(-1) of [rows, n] bf16 bits."""
    x = _u16(x)
    n = x.shape[-1]
    var = np.empty(x.size // n, np.float32)
    _check(_load().orc_rms_var(_p(x), _p(var), x.size // n, n), "rms_var")
    return var


def add_rmsnorm(x: np.ndarray, r: np.ndarray, w: np.ndarray, eps: float):
    x, r, w = _u16(x), _u16(r), _u16(w)
    n = x.shape[-1]
    normed, summed = np.empty_like(x), np.empty_like(x)
    _check(_load().orc_add_rmsnorm(_p(x), _p(r), _p(w), _p(normed), _p(summed), x.size // n,
                                   n, eps), "add_rmsnorm")
    return normed, summed


def layernorm_torch_order(n: int, aligned: bool = True) -> bool:
    """Whether eager's layer_norm takes its vectorized kernel (the restated
    Welford order): n % 4 == 0 and an 8-byte aligned contiguous input.
    Otherwise it takes its scalar row-moments kernel (order 3)."""
    return n % 4 == 0 and aligned


def layernorm(x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float,
              aligned: bool = True, stats: bool = False, _cr_recip: bool = False,
              _exact: bool = False):
    """torch layer_norm of bf16 rows; with stats=True also (mean, rstd).
    ``aligned=False`` stands for an input eager reads off 8-byte alignment.
    ``_cr_recip`` and ``_exact`` (tests only) plant mistakes: the vectorized
    order with correctly rounded reciprocals instead of gfx950's v_rcp_f32 /
    v_rsq_f32, and exactly rounded statistics instead of eager's order."""
    x, w, b = _u16(x), _u16(w), _u16(b)
    n = x.shape[-1]
    rows = x.size // n
    y = np.empty_like(x)
    mean, rstd = np.empty(rows, np.float32), np.empty(rows, np.float32)
    order = 1 if layernorm_torch_order(n, aligned) else 3
    if order == 1 and _cr_recip:
        order = 2
    if _exact:
        order = 0
    _check(_load().orc_layernorm(_p(x), _p(w), _p(b), _p(y), _p(mean), _p(rstd), rows, n, eps,
                                 order), "layernorm")
    return (y, mean, rstd) if stats else y


def ln_scalar_stats(x: np.ndarray, eps: float, variant: int):
    """(mean, rstd) of eager's scalar row-moments kernel over bf16 rows in an
    arithmetic variant (bit flags of orc_ln_scalar_stats; LN_SCALAR_EAGER is
    eager's, the others are planted mistakes for the tests)."""
    x = _u16(x)
    n = x.shape[-1]
    rows = x.size // n
    mean, rstd = np.empty(rows, np.float32), np.empty(rows, np.float32)
    _check(_load().orc_ln_scalar_stats(_p(x), _p(mean), _p(rstd), rows, n, eps, variant),
           "ln_scalar_stats")
    return mean, rstd


LN_SCALAR_EAGER = 2 | 4 | 16


def add_layernorm(x, r, w, b, eps: float):
    """bf16(x + r), then layer_norm of the rounded sum (a fresh, aligned
    tensor in eager: the vectorized kernel's order when n % 4 == 0, the
    scalar kernel's otherwise)."""
    x, r, w, b = _u16(x), _u16(r), _u16(w), _u16(b)
    n = x.shape[-1]
    normed, summed = np.empty_like(x), np.empty_like(x)
    order = 1 if layernorm_torch_order(n) else 3
    _check(_load().orc_add_layernorm(_p(x), _p(r), _p(w), _p(b), _p(normed), _p(summed),
                                     x.size // n, n, eps, order),
           "add_layernorm")
    return normed, summed


def rope_text(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x: [S, H, D] bf16 bits; cos, sin: [S, D] bf16 bits."""
    x, cos, sin = _u16(x), _u16(cos), _u16(sin)
    S, H, D = x.shape
    assert cos.shape == (S, D) and sin.shape == (S, D)
    out = np.empty_like(x)
    _load().orc_rope_text(_p(x), _p(cos), _p(sin), _p(out), S, H, D)
    return out


def rope_vision(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x: [S, H, D] bf16 bits; cos, sin: [S, D] fp32."""
    x, cos, sin = _u16(x), _f32(cos), _f32(sin)
    S, H, D = x.shape
    assert cos.shape == (S, D) and sin.shape == (S, D)
    out = np.empty_like(x)
    _load().orc_rope_vision(_p(x), _p(cos), _p(sin), _p(out), S, H, D)
    return out


def gemm_nt_f32(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """fp32(x @ w^T) with double accumulation; x [M,K], w [N,K] bf16 bits."""
    x, w = _u16(x), _u16(w)
    (M, K), (N, K2) = x.shape, w.shape
    assert K == K2
    out = np.empty((M, N), np.float32)
    _load().orc_gemm_nt_f32(_p(x), _p(w), _p(out), M, N, K)
    return out


def gate_silu_mul(x, wg, wu, fused: bool = True) -> np.ndarray:
    """silu(x @ wg^T) * (x @ wu^T); wg, wu: [N, K] bf16 bits."""
    x, wg, wu = _u16(x), _u16(wg), _u16(wu)
    (M, K), (N, K2) = x.shape, wg.shape
    assert K == K2 and wu.shape == wg.shape
    out = np.empty((M, N), np.uint16)
    _load().orc_gate_silu_mul(_p(x), _p(wg), _p(wu), _p(out), M, N, K, int(fused))
    return out


def linear(x, w, bias=None, act: int = 0, fused: bool = True) -> np.ndarray:
    """act(x @ w^T + bias); w: [N, K] bf16 bits; act 0 none / 1 erf-GELU / 2 tanh-GELU."""
    x, w = _u16(x), _u16(w)
    b = None if bias is None else _u16(bias)
    (M, K), (N, K2) = x.shape, w.shape
    assert K == K2
    out = np.empty((M, N), np.uint16)
    _load().orc_linear(_p(x), _p(w), _p(b), _p(out), M, N, K, int(act), int(fused))
    return out


def ulp_diff(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in bf16 ulps between two uint16 bf16 arrays.

    Sign-magnitude bits map to a monotone integer line (+0 and -0 both to 0),
    so adjacent representable values are 1 apart.
    """

    def ordered(v):
        v = np.asarray(v).astype(np.int32)
        neg = (v & 0x8000) != 0
        return np.where(neg, -(v & 0x7FFF), v & 0x7FFF)

    return np.abs(ordered(a) - ordered(b))
