"""GPU parity: MFMA linear (q/o projections) and fused P5 gate_silu_mul.

Small and ragged shapes are compared with the CPU oracle (double
accumulation, one rounding -- the fused kernels' own numerics); the
BASELINE shapes (M=3100, K=4096: q/o N=4096, P5 N=12288) are compared with an
fp32 torch evaluation on the same GPU.  Bar: max |err| / max |ref| <= 2e-2
and the reference's norm-relative error (scripts/check_env.py:124) <= 2e-2;
against the oracle the outputs must also agree to 1 bf16 ulp almost
everywhere (only the fp32 summation order differs).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from helpers import bf16_randn, bits, from_bits, max_rel_err, rel_err, ulp

import oracle
from umic.kernels import fused_ffn, linear

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 2e-2


def _check_vs_oracle(out, ref_bits):
    d = ulp(bits(out), ref_bits)
    assert (d <= 1).mean() > 0.999, np.bincount(d.ravel())[:8]
    ref = from_bits(ref_bits)
    assert max_rel_err(out, ref) <= TOL and rel_err(out, ref) <= TOL


@pytest.mark.parametrize("M,N,K", [(300, 520, 320), (256, 256, 64), (64, 8, 128), (1, 64, 256),
                                   (513, 1024, 512), (0, 64, 64), (130, 72, 32), (300, 264, 96)])
def test_linear_vs_oracle(M, N, K):
    g = torch.Generator().manual_seed(M + N + K)
    x, w = bf16_randn(M, K, gen=g), bf16_randn(N, K, scale=0.05, gen=g)
    y = linear.linear_hip(x.to(DEV), w.to(DEV))
    torch.cuda.synchronize()
    assert y.shape == (M, N)
    if M:
        _check_vs_oracle(y, oracle.linear(bits(x), bits(w), None, 0, fused=True))


def test_linear_bias_gelu_vs_oracle():
    g = torch.Generator().manual_seed(3)
    M, N, K = 200, 392, 192
    x, w = bf16_randn(M, K, gen=g), bf16_randn(N, K, scale=0.1, gen=g)
    b = bf16_randn(N, scale=0.5, gen=g)
    for act, code in ((None, 0), ("gelu", 1), ("gelu_tanh", 2)):
        y = linear.linear_hip(x.to(DEV), w.to(DEV), b.to(DEV), act=act)
        torch.cuda.synchronize()
        _check_vs_oracle(y, oracle.linear(bits(x), bits(w), bits(b), code, fused=True))


@pytest.mark.parametrize("act,code", [("gelu", 1), ("gelu_tanh", 2)])
def test_linear_gelu_without_bias_vs_oracle(act, code):
    g = torch.Generator().manual_seed(21)
    M, N, K = 333, 264, 256
    x, w = bf16_randn(M, K, gen=g), bf16_randn(N, K, scale=0.1, gen=g)
    y = linear.linear_hip(x.to(DEV), w.to(DEV), None, act=act)
    torch.cuda.synchronize()
    _check_vs_oracle(y, oracle.linear(bits(x), bits(w), None, code, fused=True))


def test_linear_strided_x_and_leading_dims():
    g = torch.Generator().manual_seed(4)
    big = bf16_randn(2, 70, 512 + 64, gen=g)
    w = bf16_randn(136, 512, scale=0.05, gen=g)
    x = big[..., :512]                     # row stride 576, leading dims [2, 70]
    y = linear.linear_hip(big.to(DEV)[..., :512], w.to(DEV))
    assert y.shape == (2, 70, 136)
    _check_vs_oracle(y.reshape(-1, 136), oracle.linear(bits(x.reshape(-1, 512)), bits(w), None,
                                                       0, fused=True))


@pytest.mark.parametrize("M,N,K", [(300, 520, 320), (64, 128, 64), (257, 384, 1024), (1, 8, 64),
                                   (65, 200, 160)])
def test_gate_silu_mul_vs_oracle(M, N, K):
    g = torch.Generator().manual_seed(M * 3 + N + K)
    x = bf16_randn(M, K, gen=g)
    wg, wu = bf16_randn(N, K, scale=0.05, gen=g), bf16_randn(N, K, scale=0.05, gen=g)
    y = fused_ffn.gate_silu_mul_hip(x.to(DEV), wg.to(DEV).t(), wu.to(DEV).t())
    torch.cuda.synchronize()
    _check_vs_oracle(y, oracle.gate_silu_mul(bits(x), bits(wg), bits(wu), fused=True))
    # and within the bar of the eager (bf16 per-op) chain
    eager = from_bits(oracle.gate_silu_mul(bits(x), bits(wg), bits(wu), fused=False))
    assert max_rel_err(y, eager) <= TOL and rel_err(y, eager) <= TOL


def test_gate_silu_mul_row_major_kn_weights():
    """A genuinely [K, N] row-major weight (not a .t() view) is accepted."""
    g = torch.Generator().manual_seed(5)
    x = bf16_randn(70, 128, gen=g)
    wg_kn, wu_kn = bf16_randn(128, 64, scale=0.1, gen=g), bf16_randn(128, 64, scale=0.1, gen=g)
    y = fused_ffn.gate_silu_mul(x.to(DEV), wg_kn.to(DEV), wu_kn.to(DEV))
    _check_vs_oracle(y, oracle.gate_silu_mul(bits(x), bits(wg_kn.t()), bits(wu_kn.t())))


# Shapes with fewer 256 x 256 tiles than CUs and a long K loop take the
# stream-K schedule (umic_linear_workspace_bytes > 0); on a 256-CU MI355X
# these split tiles into 2 or 3 K segments, so every reduction order (the
# last-arriving segment first, middle or last) is exercised.
SK_SHAPES = [(300, 264, 12288, 2), (700, 256, 12288, 1), (200, 392, 12288, 1)]


def _sk_bytes(M, N, K):
    from umic import _lib

    return _lib.lib().umic_linear_workspace_bytes(M, N, K)


@pytest.mark.parametrize("M,N,K,calls", SK_SHAPES)
def test_linear_stream_k_vs_oracle(M, N, K, calls):
    assert _sk_bytes(M, N, K) > 0, "shape no longer takes the stream-K schedule"
    for seed in range(calls):  # back-to-back calls reuse the stream's workspace
        g = torch.Generator().manual_seed(M + N + K + seed)
        x, w = bf16_randn(M, K, gen=g), bf16_randn(N, K, scale=0.02, gen=g)
        y = linear.linear_hip(x.to(DEV), w.to(DEV))
        torch.cuda.synchronize()
        _check_vs_oracle(y, oracle.linear(bits(x), bits(w), None, 0, fused=True))


@pytest.mark.parametrize("act,code", [("gelu", 1), ("gelu_tanh", 2)])
def test_linear_stream_k_bias_gelu_vs_oracle(act, code):
    M, N, K = 300, 264, 12288
    assert _sk_bytes(M, N, K) > 0
    g = torch.Generator().manual_seed(11)
    x, w = bf16_randn(M, K, gen=g), bf16_randn(N, K, scale=0.02, gen=g)
    b = bf16_randn(N, scale=0.5, gen=g)
    y = linear.linear_hip(x.to(DEV), w.to(DEV), b.to(DEV), act=act)
    torch.cuda.synchronize()
    _check_vs_oracle(y, oracle.linear(bits(x), bits(w), bits(b), code, fused=True))


def test_stream_k_deterministic_and_close_to_data_parallel():
    """down_proj shape (N = 4096, K = 12288) at the most rows that still take
    stream-K (176 tiles): bit-reproducible, and within fp32 summation-order
    noise of the data-parallel kernel."""
    from umic import _lib

    M, N, K = 2816, 4096, 12288
    assert _sk_bytes(M, N, K) > 0
    print(f"stream-K M={M} N={N} K={K}", flush=True)
    torch.manual_seed(5)
    x = torch.randn(M, K).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K) * 0.02).to(torch.bfloat16).to(DEV)
    y1 = linear.linear_hip(x, w)
    y2 = linear.linear_hip(x, w)
    ydp = torch.empty_like(y1)
    _lib.call("umic_linear_bf16", x.data_ptr(), w.data_ptr(), None, ydp.data_ptr(), M, N, K,
              K, K, N, 0, _lib.stream_of(x))
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    d = ulp(bits(y1), bits(ydp))
    assert (d <= 1).mean() > 0.999, np.bincount(d.ravel())[:8]
    # larger ulp counts only where the output is near zero (cancellation):
    # no difference exceeds one bf16 ulp of the largest output (2^-7 relative)
    assert ((y1.float() - ydp.float()).abs().max() / ydp.float().abs().max()).item() <= 2.0 ** -7


# Shapes with K % 64 == 0 and K >= 8192 whose tiles fill more than 11/16 of
# the CUs but leave some idle take the four-wave stream-K schedule (tails of
# every tile on the idle CUs, one or two pieces per tile, the main workgroup
# reducing): down_proj and K = 8192 at M = 3100 (208 tiles; 2-piece tiles
# and the 28-row last tile row), a shape whose tail pieces end on tile
# boundaries (192 tiles, 64 tails of exactly three tiles' tails), and ragged
# M and N (a last tile column of 160 weight rows).
W4SK_SHAPES = [(3100, 4096, 12288), (3100, 4096, 8192), (2900, 4096, 8192), (3000, 4000, 8192)]


def _dp_linear(x, w, b=None, act=0):
    from umic import _lib

    M, K = x.shape
    N = w.shape[0]
    y = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    _lib.call("umic_linear_bf16", x.data_ptr(), w.data_ptr(), _lib.ptr(b), y.data_ptr(), M, N, K,
              K, K, N, act, _lib.stream_of(x))
    return y


@pytest.mark.parametrize("M,N,K", W4SK_SHAPES)
def test_four_wave_stream_k_close_to_data_parallel(M, N, K):
    """Bit-reproducible, within fp32 summation-order noise of the
    data-parallel kernel (itself checked against the oracle), and within the
    GEMM tolerance of fp32 torch."""
    assert _sk_bytes(M, N, K) > 0
    print(f"four-wave stream-K M={M} N={N} K={K}", flush=True)
    torch.manual_seed(M + K)
    x = torch.randn(M, K).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K) * 0.02).to(torch.bfloat16).to(DEV)
    y1 = linear.linear_hip(x, w)
    y2 = linear.linear_hip(x, w)
    ydp = _dp_linear(x, w)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    d = ulp(bits(y1), bits(ydp))
    assert (d <= 1).mean() > 0.999, np.bincount(d.ravel())[:8]
    assert ((y1.float() - ydp.float()).abs().max() / ydp.float().abs().max()).item() <= 2.0 ** -7
    ref = x.float() @ w.float().t()
    assert max_rel_err(y1, ref) <= TOL


def test_four_wave_stream_k_workspace_layout():
    """The schedule's workspace: the 16,640-byte counter region (tile
    counters, status word, the few-tile schedule's slot tags), then one
    256 KB slot per tail piece, T + Gt - 1 of them, Gt = min(T, CUs - T
    rounded up to 8) rounded down to 8 tails; K below 8192 takes none."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for M, N, K in W4SK_SHAPES:
        T = -(-M // 256) * -(-N // 256)
        gt = min(T, cus - -(-T // 8) * 8) // 8 * 8
        assert _sk_bytes(M, N, K) == 16640 + (T + gt - 1) * 256 * 1024, (M, N, K)
    assert _sk_bytes(3100, 4096, 4096) == 0  # q/o: the data-parallel kernel


@pytest.mark.parametrize("act,code", [("gelu", 1), ("gelu_tanh", 2)])
def test_four_wave_stream_k_bias_gelu(act, code):
    """The bias + GELU epilogue after the partial sums, against the
    data-parallel kernel's."""
    M, N, K = 3100, 4096, 8192
    assert _sk_bytes(M, N, K) > 0
    print(f"four-wave stream-K epilogue {act}", flush=True)
    g = torch.Generator().manual_seed(17)
    x = bf16_randn(M, K, gen=g).to(DEV)
    w = bf16_randn(N, K, scale=0.02, gen=g).to(DEV)
    b = bf16_randn(N, scale=0.5, gen=g).to(DEV)
    y = linear.linear_hip(x, w, b, act=act)
    ydp = _dp_linear(x, w, b, code)
    torch.cuda.synchronize()
    d = ulp(bits(y), bits(ydp))
    assert (d <= 1).mean() > 0.999, np.bincount(d.ravel())[:8]


def test_stream_k_workspace_shared_across_shapes():
    """One stream's workspace serves stream-K calls of any shape in turn: the
    tile counters sit in a fixed region ahead of every call's partial slots,
    so a call with few tiles never stores partials where a later call with
    more tiles counts arrivals.  Shapes of 4, 176, 8, 96, 32 and 176 tiles,
    in turn, each against the data-parallel kernel."""
    from umic import _lib

    g = torch.Generator().manual_seed(13)
    for M, N, K in [(300, 264, 12288), (2816, 4096, 12288), (32, 2048, 12288),
                    (1536, 4096, 12288), (300, 4096, 12288), (2816, 4096, 12288)]:
        print(f"shared workspace: M={M} N={N} K={K}", flush=True)
        assert _sk_bytes(M, N, K) > 0
        x = bf16_randn(M, K, gen=g).to(DEV)
        w = bf16_randn(N, K, scale=0.02, gen=g).to(DEV)
        y = linear.linear_hip(x, w)
        ydp = torch.empty_like(y)
        _lib.call("umic_linear_bf16", x.data_ptr(), w.data_ptr(), None, ydp.data_ptr(), M, N, K,
                  K, K, N, 0, _lib.stream_of(x))
        torch.cuda.synchronize()
        err = ((y.float() - ydp.float()).abs().max() / ydp.float().abs().max()).item()
        assert err <= 2.0 ** -7, (M, N, K, err)


def test_down_proj_full_shape_vs_fp32():
    """BASELINE config 3 down_proj (208 tiles: the four-wave stream-K
    schedule) against fp32 torch."""
    torch.manual_seed(6)
    x = torch.randn(3100, 12288).to(torch.bfloat16).to(DEV)
    w = (torch.randn(4096, 12288) * 0.02).to(torch.bfloat16).to(DEV)
    assert _sk_bytes(3100, 4096, 12288) > 0
    y = linear.linear_hip(x, w)
    ref = x.float() @ w.float().t()
    assert max_rel_err(y, ref) <= TOL and rel_err(y, ref) <= TOL


def _fp32_ref_linear(x, w):
    return (x.float() @ w.float().t())


def test_qo_projection_full_shape():
    """q_proj / o_proj at M=3100, K=N=4096."""
    torch.manual_seed(0)
    x = torch.randn(3100, 4096).to(torch.bfloat16).to(DEV)
    w = (torch.randn(4096, 4096) * 0.02).to(torch.bfloat16).to(DEV)
    y = linear.linear_hip(x, w)
    ref = _fp32_ref_linear(x, w)
    e1, e2 = max_rel_err(y, ref), rel_err(y, ref)
    print(f"q/o proj: max_rel {e1:.2e} rel {e2:.2e}", flush=True)
    assert e1 <= TOL and e2 <= TOL


def test_p5_full_shape():
    """gate_silu_mul at M=3100, K=4096, N=12288."""
    torch.manual_seed(0)
    x = torch.randn(3100, 4096).to(torch.bfloat16).to(DEV)
    wg = (torch.randn(12288, 4096) * 0.02).to(torch.bfloat16).to(DEV)
    wu = (torch.randn(12288, 4096) * 0.02).to(torch.bfloat16).to(DEV)
    y = fused_ffn.gate_silu_mul_hip(x, wg.t(), wu.t())
    gate = x.float() @ wg.float().t()
    ref = torch.nn.functional.silu(gate) * (x.float() @ wu.float().t())
    del gate
    e1, e2 = max_rel_err(y, ref), rel_err(y, ref)
    print(f"P5: max_rel {e1:.2e} rel {e2:.2e}", flush=True)
    assert e1 <= TOL and e2 <= TOL
