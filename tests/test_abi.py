"""The C ABI surface of libumic_hip.so, checked without a GPU.

The library loads in a GPU-less process (HIP initialises lazily), exports
every function include/umic_hip.h declares with the ctypes signature the
Python side binds, and rejects bad arguments before any launch (those
paths return without touching the device).
"""

from __future__ import annotations

import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "umic_hip.h")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(umic_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from umic import _lib

    return _lib.load()


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for n in ("umic_rmsnorm_bf16", "umic_add_rmsnorm_bf16", "umic_layernorm_bf16",
              "umic_add_layernorm_bf16", "umic_rope_qk_bf16", "umic_linear_bf16",
              "umic_gate_silu_mul_bf16", "umic_linear_workspace_bytes", "umic_linear_ws_bf16",
              "umic_linear_multi_bf16", "umic_linear_add_bf16",
              "umic_rope_kv_append_bf16", "umic_qk_rmsnorm_rope_bf16",
              "umic_qk_rmsnorm_rope_kv_append_bf16", "umic_linear_sk_static_bf16",
              "umic_stream_read", "umic_stream_copy", "umic_version", "umic_error_string"):
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    from umic import _lib

    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes binding"


def test_binding_arity_matches_header():
    from umic import _lib

    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    for name, args in _lib.SIGNATURES.items():
        m = re.search(rf"\b{name}\s*\(([^)]*)\)", text)
        assert m, name
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), (name, len(params), len(args))


def test_version_and_error_strings(lib):
    from umic import _lib

    assert _lib.version().startswith("umic-hip") and "gfx950" in _lib.version()
    assert _lib.error_string(0) == "success"
    assert "invalid" in _lib.error_string(_lib.UMIC_ERR_INVALID_ARG)
    assert "unsupported" in _lib.error_string(_lib.UMIC_ERR_UNSUPPORTED)
    assert "scratch" in _lib.error_string(_lib.UMIC_ERR_SCRATCH)
    assert _lib.error_string(-99) == "unknown umic error"


def test_argument_rejection_before_launch(lib):
    """Null pointers, negative sizes and unsupported shapes return an error
    code without enqueuing anything (no device needed)."""
    from umic import _lib

    E_ARG, E_UNS = _lib.UMIC_ERR_INVALID_ARG, _lib.UMIC_ERR_UNSUPPORTED
    fake = 1 << 20  # never dereferenced: every call below fails validation
    assert lib.umic_rmsnorm_bf16(None, fake, fake, 4, 64, 64, 64, 1e-6, None) == E_ARG
    assert lib.umic_rmsnorm_bf16(fake, fake, fake, -1, 64, 64, 64, 1e-6, None) == E_ARG
    assert lib.umic_rmsnorm_bf16(fake, fake, fake, 4, 64, 32, 64, 1e-6, None) == E_ARG
    assert lib.umic_rmsnorm_bf16(fake, fake, fake, 0, 64, 64, 64, 1e-6, None) == 0
    # empty tensors carry null data pointers in torch: accepted, nothing launched
    assert lib.umic_rmsnorm_bf16(None, None, None, 0, 64, 64, 64, 1e-6, None) == 0
    assert lib.umic_add_layernorm_bf16(None, None, None, None, None, None, 0, 64, 64, 64, 64,
                                       64, 1e-6, None) == 0
    assert lib.umic_linear_bf16(None, None, None, None, 0, 64, 128, 128, 128, 64, 0, None) == 0
    assert lib.umic_gate_silu_mul_bf16(None, None, None, None, 0, 64, 128, 128, 128, 128, 64,
                                       None) == 0
    assert lib.umic_add_rmsnorm_bf16(fake, None, fake, fake, fake, 4, 64, 64, 64, 64, 64,
                                     1e-6, None) == E_ARG
    assert lib.umic_layernorm_bf16(fake, fake, None, fake, 4, 64, 64, 64, 1e-6, None) == E_ARG
    # linear: K not a multiple of 32, N not a multiple of 8, bad act
    assert lib.umic_linear_bf16(fake, fake, None, fake, 8, 64, 80, 80, 80, 64, 0, None) == E_UNS
    assert lib.umic_linear_bf16(fake, fake, None, fake, 8, 60, 128, 128, 128, 60, 0, None) == E_UNS
    assert lib.umic_linear_bf16(fake, fake, None, fake, 8, 64, 128, 128, 128, 64, 7, None) == E_ARG
    assert lib.umic_linear_bf16(fake, fake, None, fake, 8, 64, 128, 128, 128, 64, 3, None) == E_ARG
    assert lib.umic_linear_bf16(fake, fake, None, fake, 0, 64, 128, 128, 128, 64, 0, None) == 0
    # the static-scratch stream-K linear checks its arguments the same way
    sk = lib.umic_linear_sk_static_bf16
    assert sk(None, None, None, None, 0, 64, 128, 128, 128, 64, 0, None) == 0
    assert sk(None, fake, None, fake, 300, 4096, 12288, 12288, 12288, 4096, 0, None) == E_ARG
    assert sk(fake, fake, None, fake, -1, 64, 128, 128, 128, 64, 0, None) == E_ARG
    assert sk(fake, fake, None, fake, 300, 4096, 12288, 12288, 12288, 4096, 3, None) == E_ARG
    assert sk(fake, fake, None, fake, 300, 4092, 12288, 12288, 12288, 4092, 0, None) == E_UNS
    assert sk(fake, fake, fake + 2, fake, 300, 4096, 12288, 12288, 12288, 4096, 0, None) == E_UNS
    # the read-ceiling helper: negative / misaligned sizes and pointers
    rd = lib.umic_stream_read
    assert rd(fake, -16, fake, None) == E_ARG
    assert rd(None, 0, None, None) == 0
    assert rd(None, 4096, fake, None) == E_ARG
    assert rd(fake, 4100, fake, None) == E_UNS
    assert rd(fake + 8, 4096, fake, None) == E_UNS
    # the copy-ceiling helper: the same, and overlapping ranges
    cp = lib.umic_stream_copy
    assert cp(fake, fake + 8192, -16, None) == E_ARG
    assert cp(None, None, 0, None) == 0
    assert cp(None, fake, 4096, None) == E_ARG
    assert cp(fake, fake + 2048, 4096, None) == E_ARG
    assert cp(fake + 4096, fake, 4096 + 16, None) == E_ARG
    assert cp(fake, fake + 8192, 4100, None) == E_UNS
    assert cp(fake, fake + 8200, 4096, None) == E_UNS
    assert lib.umic_gate_silu_mul_bf16(fake, fake, None, fake, 8, 64, 128, 128, 128, 128, 64,
                                       None) == E_ARG
    # stream-K linear: same validation; a negative workspace size is rejected
    assert lib.umic_linear_workspace_bytes(0, 64, 128) == 0
    assert lib.umic_linear_workspace_bytes(64, 64, 100) == 0  # K not a multiple of 32
    assert lib.umic_linear_ws_bf16(fake, fake, None, fake, 8, 64, 80, 80, 80, 64, 0, None, 0,
                                   None) == E_UNS
    assert lib.umic_linear_ws_bf16(fake, fake, None, fake, 8, 64, 128, 128, 128, 64, 7, None, 0,
                                   None) == E_ARG
    assert lib.umic_linear_ws_bf16(fake, fake, None, fake, 8, 64, 128, 128, 128, 64, 0, fake, -1,
                                   None) == E_ARG
    assert lib.umic_linear_ws_bf16(None, None, None, None, 0, 64, 128, 128, 128, 64, 0, None, 0,
                                   None) == 0
    # rope: odd head dim, text mode with fp32 tables, bad mode
    args = [fake, fake, fake, fake, fake, fake]
    strides = [0] * 12 + [0, 0]
    assert lib.umic_rope_qk_bf16(*args, 0, 0, 1, 4, 2, 2, 81, *strides, None) == E_UNS
    assert lib.umic_rope_qk_bf16(*args, 1, 0, 1, 4, 2, 2, 64, *strides, None) == E_UNS
    assert lib.umic_rope_qk_bf16(*args, 0, 5, 1, 4, 2, 2, 64, *strides, None) == E_ARG
    assert lib.umic_rope_qk_bf16(*args, 0, 0, 1, 0, 2, 2, 64, *strides, None) == 0
    # rope + KV append: q, k, v, q_out, k_cache, v_cache, cos, sin; then
    # B, S, Hq, Hk, D, 12 strides, 3 cache strides, capacity, pos, pos_dev,
    # 2 table strides
    kv = [fake] * 8
    st = [8] * 12 + [8, 8, 8]
    ok = lambda S, D, cap, pos, pos_dev=None, ptrs=kv: lib.umic_rope_kv_append_bf16(  # noqa: E731
        *ptrs, 1, S, 4, 2, D, *st, cap, pos, pos_dev, 8, 8, None)
    assert ok(4, 128, 16, 13) == E_ARG            # pos + S past the cache (reference raises)
    assert ok(4, 128, 16, -1) == E_ARG            # negative position
    assert ok(4, 120, 16, 0) == E_UNS             # D not a multiple of 16
    assert ok(4, 128, -1, 0) == E_ARG             # negative capacity
    assert ok(4, 128, 16, 0, ptrs=[fake] * 5 + [None] + [fake] * 2) == E_ARG  # no v cache
    assert ok(0, 128, 16, 0, ptrs=[None] * 8) == 0   # empty: nothing launched


def test_qk_norm_rope_rejection(lib):
    """Argument checks of the fused q/k RMSNorm + RoPE entry points, before
    any launch (no GPU needed): bad sizes, head dims the row group cannot
    take, missing weights, misalignment; empty inputs are no-ops."""
    E_ARG, E_UNS = -1, -2
    f = lib.umic_qk_rmsnorm_rope_bf16
    fake = 1 << 20   # 16-byte aligned, never dereferenced: every case returns early
    strides = [1024, 1024, 128] * 4
    assert f(None, None, None, None, None, None, 1e-6, None, None, 1, 0, 4, 1, 128,
             *strides, 128, 128, None) == 0                             # S = 0: no-op
    assert f(fake, fake, fake, fake, fake, fake, 1e-6, fake, fake, -1, 4, 4, 1, 128,
             *strides, 128, 128, None) == E_ARG
    assert f(fake, fake, fake, fake, fake, fake, 1e-6, fake, fake, 1, 4, 4, 1, 96,
             *strides, 128, 128, None) == E_UNS                         # 96/16 = 6
    assert f(fake, fake, fake, fake, fake, fake, 1e-6, fake, fake, 1, 4, 4, 1, 136,
             *strides, 128, 128, None) == E_UNS                         # 136 % 16
    assert f(fake, fake, fake, fake, None, fake, 1e-6, fake, fake, 1, 4, 4, 1, 128,
             *strides, 128, 128, None) == E_ARG                         # no q weight
    assert f(fake + 2, fake, fake, fake, fake, fake, 1e-6, fake, fake, 1, 4, 4, 1, 128,
             *strides, 128, 128, None) == E_UNS                         # misaligned q
    g = lib.umic_qk_rmsnorm_rope_kv_append_bf16
    kv = [1024, 1024, 128] * 4 + [4096, 4096, 128]
    assert g(fake, fake, fake, fake, fake, fake, fake, fake, fake, fake, 1e-6, 1, 4, 4, 1, 128,
             *kv[:12], 8 * 4096 * 128, 4096 * 128, 128, 100, 98, None, 128, 128,
             None) == E_ARG                                             # 98 + 4 > 100
    assert g(fake, fake, fake, fake, fake, fake, fake, fake, fake, None, 1e-6, 1, 4, 4, 1, 128,
             *kv[:12], 8 * 4096 * 128, 4096 * 128, 128, 100, 0, None, 128, 128,
             None) == E_ARG                                             # no k weight
    assert g(fake, fake, fake, fake, fake, fake, fake, fake, fake, fake, 1e-6, 1, 4, 4, 1, 80,
             *kv[:12], 8 * 4096 * 80, 4096 * 80, 80, 100, 0, None, 80, 80,
             None) == E_UNS                                             # 80/16 = 5


def test_linear_multi_rejection(lib):
    """Argument checks of the multi-linear decode GEMV, before any launch."""
    import ctypes

    E_ARG, E_UNS = -1, -2
    f = lib.umic_linear_multi_bf16
    fake = 1 << 20
    P3 = ctypes.c_void_p * 3
    I3 = ctypes.c_int64 * 3
    w, out = P3(fake, fake, fake), P3(fake, fake, fake)
    N, ldw, ldo = I3(64, 16, 16), I3(128, 128, 128), I3(64, 16, 16)
    assert f(fake, 0, 128, 128, 3, w, None, out, N, ldw, ldo, 0, None) == 0   # M = 0: no-op
    assert f(fake, 1, 128, 128, 0, w, None, out, N, ldw, ldo, 0, None) == E_ARG
    assert f(fake, 1, 128, 128, 4, w, None, out, N, ldw, ldo, 0, None) == E_ARG
    assert f(fake, 1, 128, 128, 3, w, None, out, N, ldw, ldo, 5, None) == E_ARG  # act
    assert f(fake, 9, 128, 128, 3, w, None, out, N, ldw, ldo, 0, None) == E_UNS  # not decode
    assert f(fake, 1, 80, 128, 3, w, None, out, N, ldw, ldo, 0, None) == E_UNS   # K % 32
    assert f(fake, 1, 128, 128, 3, w, None, out, I3(64, -1, 16), ldw, ldo, 0, None) == E_ARG
    assert f(fake, 1, 128, 128, 3, w, None, out, N, I3(128, 64, 128), ldo, 0, None) == E_ARG
    assert f(fake, 1, 128, 128, 3, P3(fake, fake + 2, fake), None, out, N, ldw, ldo, 0,
             None) == E_UNS                                             # misaligned w


def test_linear_add_rejection(lib):
    E_ARG, E_UNS = -1, -2
    f = lib.umic_linear_add_bf16
    fake = 1 << 20
    assert f(fake, fake, None, fake, fake, 0, 64, 128, 128, 128, 64, 64, None) == 0  # M = 0
    assert f(fake, fake, None, fake, fake, 9, 64, 128, 128, 128, 64, 64, None) == E_UNS
    assert f(fake, fake, None, None, fake, 1, 64, 128, 128, 128, 64, 64, None) == E_ARG
    assert f(fake, fake, None, fake, fake, 1, 64, 128, 128, 128, 32, 64, None) == E_ARG  # ldr
    assert f(fake, fake, None, fake, fake, 1, 64, 80, 128, 128, 64, 64, None) == E_UNS   # K % 32


def test_wrappers_refuse_cpu_tensors():
    import torch

    from umic.kernels import layernorm, linear, rmsnorm

    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    w = torch.ones(64, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        rmsnorm.rmsnorm_hip(x, w, 1e-6)
    with pytest.raises(ValueError):
        layernorm.layernorm_hip(x, w, w, 1e-6)
    with pytest.raises(ValueError):
        linear.linear_hip(x, torch.zeros(64, 64, dtype=torch.bfloat16))


def test_missing_library_fails_loudly(monkeypatch):
    """With the library unloadable, loading raises UmicLibraryError (the
    wrappers call it before any launch)."""
    from umic import _lib

    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "HAS_KERNELS", False)
    with pytest.raises(_lib.UmicLibraryError):
        _lib.load("/nonexistent/libumic_hip.so")
    assert not _lib.HAS_KERNELS
