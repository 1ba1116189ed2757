"""ctypes binding of libumic_hip.so, the gfx950 kernel library.

The C ABI (``include/umic_hip.h``) takes raw device pointers, sizes and a
``hipStream_t``; this module owns the one process-wide handle to it and the
glue every wrapper needs: argument marshalling, the current-stream handle
and return-code checking.  torch is used only as the allocator and stream
owner -- no torch types cross the boundary.

``HAS_KERNELS`` is True once the library has loaded (it loads lazily on first
use, or eagerly via :func:`load`).  A wrapper called on device tensors while
the library is missing raises :class:`UmicLibraryError`; the injection layer
checks :func:`available` first and patches nothing when it is False.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libumic_hip.so")

UMIC_OK = 0
UMIC_ERR_INVALID_ARG = -1
UMIC_ERR_UNSUPPORTED = -2
UMIC_ERR_SCRATCH = -3
UMIC_ROPE_TEXT = 0
UMIC_ROPE_VISION = 1
UMIC_ACT_NONE = 0
UMIC_ACT_GELU = 1
UMIC_ACT_GELU_TANH = 2
UMIC_STREAM_READ_GRID = 2048  # fold words umic_stream_read writes

_P, _I64, _F32, _I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int

# Exported function -> argument types, exactly as declared in umic_hip.h.
SIGNATURES: dict[str, list] = {
    "umic_rmsnorm_bf16": [_P, _P, _P, _I64, _I64, _I64, _I64, _F32, _P],
    "umic_add_rmsnorm_bf16": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F32, _P],
    "umic_layernorm_bf16": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _F32, _P],
    "umic_add_layernorm_bf16": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                                _F32, _P],
    "umic_rope_qk_bf16": [_P, _P, _P, _P, _P, _P, _I, _I] + [_I64] * 5 + [_I64] * 12
                         + [_I64] * 2 + [_P],
    "umic_rope_kv_append_bf16": [_P] * 8 + [_I64] * 5 + [_I64] * 12 + [_I64] * 4
                                + [_I64, _P] + [_I64] * 2 + [_P],
    "umic_qk_rmsnorm_rope_bf16": [_P] * 6 + [_F32] + [_P] * 2 + [_I64] * 5 + [_I64] * 12
                                 + [_I64] * 2 + [_P],
    "umic_qk_rmsnorm_rope_kv_append_bf16": [_P] * 10 + [_F32] + [_I64] * 5 + [_I64] * 12
                                           + [_I64] * 4 + [_I64, _P] + [_I64] * 2 + [_P],
    "umic_linear_bf16": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P],
    "umic_linear_multi_bf16": [_P, _I64, _I64, _I64, _I] + [_P] * 6 + [_I, _P],
    "umic_linear_add_bf16": [_P] * 5 + [_I64] * 7 + [_P],
    "umic_gate_silu_mul_bf16": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    "umic_rmsnorm_linear_multi_bf16": [_P, _P, _P, _I64, _I64, _I64, _I64, _F32, _I]
                                      + [_P] * 6 + [_P],
    "umic_add_rmsnorm_gate_silu_mul_bf16": [_P] * 8 + [_I64] * 10 + [_F32, _P],
    "umic_linear_workspace_bytes": [_I64, _I64, _I64],
    "umic_linear_ws_bf16": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P, _I64, _P],
    "umic_linear_sk_static_bf16": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P],
    "umic_stream_read": [_P, _I64, _P, _P],
    "umic_stream_copy": [_P, _P, _I64, _P],
    "umic_version": [],
    "umic_error_string": [_I],
}


# Return types other than int.
RESTYPES = {"umic_version": ctypes.c_char_p, "umic_error_string": ctypes.c_char_p,
            "umic_linear_workspace_bytes": _I64}


class UmicLibraryError(RuntimeError):
    """libumic_hip.so is missing or failed to load while a kernel was needed."""


class UmicKernelError(RuntimeError):
    """A libumic_hip.so entry point returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with code {code}: {msg}")
        self.code = code


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_load_error: str | None = None
_fns: dict[str, object] = {}   # entry-point name -> ctypes function of _lib
HAS_KERNELS = False


def load(path: str | None = None) -> ctypes.CDLL:
    """Load the library (idempotent) and return the ctypes handle."""
    global _lib, _load_error, HAS_KERNELS
    with _lock:
        if _lib is not None:
            return _lib
        p = path or os.environ.get("UMIC_HIP_LIB", LIB_PATH)
        try:
            lib = ctypes.CDLL(p)
        except OSError as exc:
            _load_error = f"cannot load {p}: {exc}"
            raise UmicLibraryError(_load_error) from exc
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = RESTYPES.get(name, _I)
        _lib = lib
        _fns.clear()
        HAS_KERNELS = True
        return lib


def available() -> bool:
    """True if the library is (or can be) loaded."""
    if _lib is not None:
        return True
    try:
        load()
        return True
    except UmicLibraryError:
        return False


def load_error() -> str | None:
    """Why the last load attempt failed (None if it has not failed)."""
    return _load_error


def lib() -> ctypes.CDLL:
    if _lib is not None:
        return _lib
    return load()


def version() -> str:
    return lib().umic_version().decode()


def error_string(code: int) -> str:
    return lib().umic_error_string(code).decode()


def call(name: str, *args) -> None:
    """Invoke entry point ``name``; raise UmicKernelError on non-zero status."""
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(lib(), name)
    rc = fn(*args)
    if rc != UMIC_OK:
        raise UmicKernelError(name, rc, error_string(rc))


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# torch's accessor for the raw handle of a device's current stream (what
# torch.cuda.current_stream(dev).cuda_stream returns, without building a
# Stream object: ~0.1 us against ~2 us per call); the public path otherwise.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t handle of the current torch stream on t's device."""
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


class device_of:
    """Make t's device current for the duration of a launch (no-op if it is)."""

    def __init__(self, t: torch.Tensor):
        self.idx = t.device.index
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if self.idx is not None and cur != self.idx:
            self.prev = cur
            torch.cuda.set_device(self.idx)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


def aligned16(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0
