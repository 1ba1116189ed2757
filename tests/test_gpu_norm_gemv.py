"""GPU: the decode launches that fold an RMSNorm into the GEMV consuming it.

umic_rmsnorm_linear_multi_bf16 (input_layernorm + q/k/v) and
umic_add_rmsnorm_gate_silu_mul_bf16 (residual add + post_attention_layernorm
+ P5) must equal, bit for bit, the two launches they replace -- the library's
RMSNorm kernels (bit-exact against torch-ROCm eager, tests/test_gpu_norm.py)
followed by its GEMVs -- and the oracle's composition of the same steps.  The
host-side plan test (rmsnorm.gemv_norm_ok) must agree with what the library
accepts.  Then a BASELINE config-5 decoder layer at decode: the folded path
against the same fused layer with folding switched off, bit for bit.
"""

from __future__ import annotations

import collections
import ctypes

import numpy as np
import pytest
import torch
from helpers import bf16_randn, bits, qwen3_decoder_layer, ulp

import oracle
from umic import _lib, integrate
from umic.kernels import fused_ffn, linear, rmsnorm

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::FutureWarning")]
DEV = "cuda"
EPS = 1e-6


def _norm_w(K, g):
    return (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16)


@pytest.mark.parametrize("M,K,Ns", [(1, 4096, (4096, 1024, 1024)), (2, 4096, (256, 64)),
                                    (1, 2048, (520,)), (2, 512, (64, 8, 16)),
                                    (1, 3072, (128,)), (2, 2016, (72,)), (1, 640, (8, 8))])
def test_rmsnorm_linear_multi_equals_two_launches(M, K, Ns):
    print(f"norm + multi-linear M={M} K={K} N={Ns}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + K)
    x = bf16_randn(M, K, gen=g).to(DEV)
    nw = _norm_w(K, g).to(DEV)
    ws = [bf16_randn(N, K, scale=0.02, gen=g).to(DEV) for N in Ns]
    bs = [bf16_randn(N, scale=0.5, gen=g).to(DEV) if i == 1 else None for i, N in enumerate(Ns)]
    assert rmsnorm.gemv_norm_ok(M, K)
    got = linear.rmsnorm_linear_multi_hip(x, nw, EPS, ws, bs)
    y = rmsnorm.rmsnorm_hip(x, nw, EPS)
    ref = linear.linear_multi_hip(y, ws, bs)
    # the optional normed output
    normed = torch.empty_like(x)
    n = len(ws)
    P, I64 = ctypes.c_void_p * n, ctypes.c_int64 * n
    outs = [torch.empty(M, N, dtype=torch.bfloat16, device=DEV) for N in Ns]
    _lib.call("umic_rmsnorm_linear_multi_bf16", x.data_ptr(), nw.data_ptr(), normed.data_ptr(),
              M, K, K, K, EPS, n, P(*[w.data_ptr() for w in ws]),
              P(*[_lib.ptr(b) for b in bs]), P(*[o.data_ptr() for o in outs]), I64(*Ns),
              I64(*[K] * n), I64(*Ns), _lib.stream_of(x))
    torch.cuda.synchronize()
    assert torch.equal(normed, y)
    for a, b, c in zip(got, ref, outs):
        assert torch.equal(a, b) and torch.equal(c, b)
    # the oracle's composition: its RMSNorm, then its linear
    yo = oracle.rmsnorm(bits(x), bits(nw), EPS)
    assert np.array_equal(bits(y), yo)
    for w, b, o in zip(ws, bs, got):
        ro = oracle.linear(yo, bits(w), None if b is None else bits(b), 0, fused=True)
        d = ulp(bits(o), ro)
        assert (d <= 1).mean() > 0.999, np.bincount(d.ravel())[:4]


@pytest.mark.parametrize("M,N,K", [(1, 12288, 4096), (2, 1024, 4096), (1, 64, 512),
                                   (2, 136, 2048)])
def test_add_rmsnorm_gate_silu_mul_equals_two_launches(M, N, K):
    print(f"add + norm + P5 M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M * 11 + N + K)
    x = bf16_randn(M, K, gen=g).to(DEV)
    r = bf16_randn(M, K, gen=g).to(DEV)
    nw = _norm_w(K, g).to(DEV)
    wg = bf16_randn(N, K, scale=0.02, gen=g).to(DEV)
    wu = bf16_randn(N, K, scale=0.02, gen=g).to(DEV)
    out, summed = fused_ffn.add_rmsnorm_gate_silu_mul_hip(x, r, nw, EPS, wg.t(), wu.t())
    y, s = rmsnorm.add_rmsnorm_hip(x, r, nw, EPS)
    ref = fused_ffn.gate_silu_mul_hip(y, wg.t(), wu.t())
    normed = torch.empty_like(x)
    out2 = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    _lib.call("umic_add_rmsnorm_gate_silu_mul_bf16", x.data_ptr(), r.data_ptr(), nw.data_ptr(),
              normed.data_ptr(), None, wg.data_ptr(), wu.data_ptr(), out2.data_ptr(), M, N, K,
              K, K, K, K, K, K, N, EPS, _lib.stream_of(x))
    torch.cuda.synchronize()
    assert torch.equal(out, ref) and torch.equal(out2, ref)
    assert torch.equal(summed, s) and torch.equal(normed, y)
    yo, so = oracle.add_rmsnorm(bits(x), bits(r), bits(nw), EPS)
    assert np.array_equal(bits(y), yo) and np.array_equal(bits(s), so)
    ro = oracle.gate_silu_mul(yo, bits(wg), bits(wu), fused=True)
    d = ulp(bits(out), ro)
    assert (d <= 1).mean() > 0.999, np.bincount(d.ravel())[:4]


@pytest.mark.parametrize("M", [1, 2, 3])
def test_plan_agrees_with_the_library(M):
    """gemv_norm_ok(M, K), with the GEMV's own K rule, is True exactly where
    the library takes the call."""
    g = torch.Generator().manual_seed(3)
    w = bf16_randn(8, 8192, scale=0.02, gen=g).to(DEV)
    xfull = bf16_randn(3, 8192, gen=g).to(DEV)
    nw = _norm_w(8192, g).to(DEV)
    out = torch.empty(3, 8, dtype=torch.bfloat16, device=DEV)
    P, I64 = ctypes.c_void_p * 1, ctypes.c_int64 * 1
    fn = _lib.lib().umic_rmsnorm_linear_multi_bf16
    for K in (256, 504, 512, 640, 1024, 3072, 4096, 4608, 7680, 7936, 8192):
        rc = fn(xfull.data_ptr(), nw.data_ptr(), None, M, K, 8192, K, ctypes.c_float(EPS), 1,
                P(w.data_ptr()), P(None), P(out.data_ptr()), I64(8), I64(8192), I64(8),
                ctypes.c_void_p(_lib.stream_of(xfull)))
        assert rc in (_lib.UMIC_OK, _lib.UMIC_ERR_UNSUPPORTED), (M, K, rc)
        ok = rmsnorm.gemv_norm_ok(M, K) and K % linear.K_MULTIPLE == 0
        assert (rc == _lib.UMIC_OK) == ok, (M, K, rc)
    torch.cuda.synchronize()


def test_outputs_overlapping_inputs_are_rejected():
    g = torch.Generator().manual_seed(4)
    x = bf16_randn(1, 4096, gen=g).to(DEV)
    r = bf16_randn(1, 4096, gen=g).to(DEV)
    nw = _norm_w(4096, g).to(DEV)
    w = bf16_randn(64, 4096, scale=0.02, gen=g).to(DEV)
    out = torch.empty(1, 64, dtype=torch.bfloat16, device=DEV)
    P, I64 = ctypes.c_void_p * 1, ctypes.c_int64 * 1
    rc = _lib.lib().umic_rmsnorm_linear_multi_bf16(
        x.data_ptr(), nw.data_ptr(), x.data_ptr(), 1, 4096, 4096, 4096, ctypes.c_float(EPS), 1,
        P(w.data_ptr()), P(None), P(out.data_ptr()), I64(64), I64(4096), I64(64),
        ctypes.c_void_p(_lib.stream_of(x)))
    assert rc == _lib.UMIC_ERR_INVALID_ARG
    for normed, summed in ((None, r), (x, None)):
        rc = _lib.lib().umic_add_rmsnorm_gate_silu_mul_bf16(
            x.data_ptr(), r.data_ptr(), nw.data_ptr(), _lib.ptr(normed), _lib.ptr(summed),
            w.data_ptr(), w.data_ptr(), out.data_ptr(), 1, 64, 4096, 4096, 4096, 4096, 4096,
            4096, 4096, 64, ctypes.c_float(EPS), ctypes.c_void_p(_lib.stream_of(x)))
        assert rc == _lib.UMIC_ERR_INVALID_ARG
    torch.cuda.synchronize()


def test_decoder_layer_decode_folds_both_norms(monkeypatch):
    """Config-5 layer at decode (one row, DynamicCache after a 64-token
    prefill) with every fusion applied: input_layernorm rides in the q/k/v
    GEMV and the post-attention add + norm in the P5 GEMV, and the output is
    bit-identical to the same fused layer with folding switched off."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    from transformers.cache_utils import DynamicCache

    layer, rot = qwen3_decoder_layer(DEV)
    torch.manual_seed(12)
    P = 64
    h0 = torch.randn(1, P, 4096).to(torch.bfloat16).to(DEV)
    x = torch.randn(1, 1, 4096).to(torch.bfloat16).to(DEV)
    log = collections.Counter()
    real = _lib.call

    def spy(name, *args):
        log[name] += 1
        return real(name, *args)

    try:
        with torch.no_grad(), sdpa_kernel([SDPBackend.FLASH_ATTENTION,
                                           SDPBackend.EFFICIENT_ATTENTION]):
            assert integrate.fuse_mlps(layer) == 1 and integrate.fuse_linears(layer) == 2
            assert integrate.fuse_rmsnorms(layer) == 4 and integrate.fuse_add_rmsnorm(layer) == 1
            assert integrate.fuse_text_rope() and integrate.fuse_kv_rope(layer) == 1
            outs = {}
            for fold in (False, True):
                cache = DynamicCache()
                layer(h0, position_embeddings=rot(h0, torch.arange(P, device=DEV)[None]),
                      past_key_values=cache)
                cs = rot(x, torch.tensor([[P]], device=DEV))
                with monkeypatch.context() as mp:
                    if not fold:
                        mp.setattr(rmsnorm, "gemv_norm_ok", lambda *a: False)
                    mp.setattr(_lib, "call", spy)
                    log.clear()
                    outs[fold] = layer(x, position_embeddings=cs, past_key_values=cache)
                    torch.cuda.synchronize()
                calls = dict(log)
                print(f"decode fold={fold}: calls {calls}", flush=True)
                if fold:
                    assert log["umic_rmsnorm_linear_multi_bf16"] == 1
                    assert log["umic_add_rmsnorm_gate_silu_mul_bf16"] == 1
                    for name in ("umic_rmsnorm_bf16", "umic_add_rmsnorm_bf16",
                                 "umic_linear_multi_bf16", "umic_gate_silu_mul_bf16"):
                        assert log[name] == 0, name
                else:
                    assert log["umic_rmsnorm_linear_multi_bf16"] == 0
                    assert log["umic_linear_multi_bf16"] == 1
                    assert log["umic_add_rmsnorm_bf16"] == 1
        assert torch.equal(outs[True], outs[False])
    finally:
        integrate.unfuse_rope()
        integrate.unfuse_mlps(layer)


def test_folded_decode_step_in_a_captured_graph():
    """The folded decode step of a config-5 layer (no cache) captured in one
    HIP graph: four replays, with eager work and synchronisations between
    them, equal the eager fused step bit for bit."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    layer, rot = qwen3_decoder_layer(DEV)
    torch.manual_seed(13)
    x = torch.randn(1, 1, 4096).to(torch.bfloat16).to(DEV)
    cs = rot(x, torch.tensor([[5]], device=DEV))
    try:
        with torch.no_grad(), sdpa_kernel([SDPBackend.FLASH_ATTENTION,
                                           SDPBackend.EFFICIENT_ATTENTION]):
            assert integrate.fuse_mlps(layer) == 1 and integrate.fuse_linears(layer) == 2
            assert integrate.fuse_rmsnorms(layer) == 4 and integrate.fuse_add_rmsnorm(layer) == 1
            assert integrate.fuse_text_rope() and integrate.fuse_kv_rope(layer) == 1
            ref = layer(x, position_embeddings=cs)
            torch.cuda.synchronize()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                layer(x, position_embeddings=cs)
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                out = layer(x, position_embeddings=cs)
            for i in range(4):
                print(f"folded decode graph replay {i}", flush=True)
                graph.replay()
                torch.cuda.synchronize()
                assert torch.equal(out, ref), i
                _ = (x.float() * 2).sum().item()  # eager work between replays
    finally:
        integrate.unfuse_rope()
        integrate.unfuse_mlps(layer)
