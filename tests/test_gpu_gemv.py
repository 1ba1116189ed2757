"""GPU parity: the few-row (decode) GEMV path behind umic_linear_bf16 and
umic_gate_silu_mul_bf16 (M <= 8 rows).

Small and ragged shapes against the CPU oracle (double accumulation, one
rounding; the GEMV's fp32 lane sums differ only in order, so the outputs
agree to one bf16 ulp almost everywhere), K values whose 16-byte chunk
count is not a multiple of the 64-lane slab (a partial last slab), every
row count 1..8 (the kernel pads to 1, 2, 4 or 8 rows), the bias and both
GELU epilogues, a strided x, and the config-5 decode shapes (q / k / o
projections, P5 gate/up, down_proj) against an fp32 torch evaluation on the
same GPU.  Bar: max |err| / max |ref| <= 2e-2 and the norm-relative error
<= 2e-2.
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


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("N,K", [(264, 1056), (8, 32), (1024, 4096)])
def test_gemv_linear_vs_oracle(M, N, K):
    print(f"gemv linear M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + N + K)
    x, w = bf16_randn(M, K, gen=g), bf16_randn(N, K, scale=0.05, gen=g)
    y = linear.linear_hip(x.to(DEV), w.to(DEV))
    torch.cuda.synchronize()
    assert y.shape == (M, N)
    _check_vs_oracle(y, oracle.linear(bits(x), bits(w), None, 0, fused=True))


@pytest.mark.parametrize("M", [1, 6])
def test_gemv_bias_and_gelu_vs_oracle(M):
    g = torch.Generator().manual_seed(40 + M)
    N, K = 392, 192
    x, w = bf16_randn(M, K, gen=g), bf16_randn(N, K, scale=0.1, gen=g)
    b = bf16_randn(N, scale=0.5, gen=g)
    for act, code in ((None, 0), ("gelu", 1), ("gelu_tanh", 2)):
        y = linear.linear_hip(x.to(DEV), w.to(DEV), b.to(DEV), act=act)
        torch.cuda.synchronize()
        _check_vs_oracle(y, oracle.linear(bits(x), bits(w), bits(b), code, fused=True))


def test_gemv_strided_x():
    """x rows at a leading dim larger than K (a column slice of a wider
    tensor) and an odd row count."""
    g = torch.Generator().manual_seed(9)
    M, N, K = 3, 136, 512
    wide = bf16_randn(M, K + 64, gen=g)
    w = bf16_randn(N, K, scale=0.05, gen=g)
    x = wide.to(DEV)[:, 32:32 + K]
    assert x.stride(0) == K + 64
    y = linear.linear_hip(x, w.to(DEV))
    torch.cuda.synchronize()
    _check_vs_oracle(y, oracle.linear(bits(wide[:, 32:32 + K]), bits(w), None, 0, fused=True))


@pytest.mark.parametrize("M", [1, 3, 8])
def test_gemv_gate_silu_mul_vs_oracle(M):
    print(f"gemv gate_silu_mul M={M}", flush=True)
    g = torch.Generator().manual_seed(60 + M)
    N, K = 520, 1056
    x = bf16_randn(M, K, gen=g)
    wg, wu = bf16_randn(N, K, scale=0.05, gen=g), bf16_randn(N, K, scale=0.05, gen=g)
    y = fused_ffn.gate_silu_mul_hip(x.to(DEV), wg.to(DEV).t(), wu.to(DEV).t())
    torch.cuda.synchronize()
    _check_vs_oracle(y, oracle.gate_silu_mul(bits(x), bits(wg), bits(wu), fused=True))


def test_gemv_and_tiled_agree_at_the_boundary():
    """8 rows run the GEMV, 9 the tiled kernel; the first 8 rows of the 9-row
    product equal the 8-row product to one bf16 ulp almost everywhere."""
    g = torch.Generator().manual_seed(77)
    N, K = 1024, 4096
    x9, w = bf16_randn(9, K, gen=g).to(DEV), bf16_randn(N, K, scale=0.02, gen=g).to(DEV)
    y8 = linear.linear_hip(x9[:8], w)
    y9 = linear.linear_hip(x9, w)
    torch.cuda.synchronize()
    d = ulp(bits(y8), bits(y9[:8]))
    assert (d <= 1).mean() > 0.999
    assert max_rel_err(y8, y9[:8]) <= TOL and rel_err(y8, y9[:8]) <= TOL


@pytest.mark.parametrize("site,N,K", [("q_proj", 4096, 4096), ("k_proj", 1024, 4096),
                                      ("down_proj", 4096, 12288)])
def test_gemv_decode_shapes_vs_fp32(site, N, K):
    print(f"gemv decode {site} N={N} K={K}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(N + K)
    x = torch.randn(1, K, generator=g, device=DEV).to(torch.bfloat16)
    w = (0.02 * torch.randn(N, K, generator=g, device=DEV)).to(torch.bfloat16)
    y = linear.linear_hip(x, w)
    ref = x.float() @ w.float().t()
    torch.cuda.synchronize()
    e1, e2 = max_rel_err(y, ref), rel_err(y, ref)
    print(f"  max_rel {e1:.2e} rel {e2:.2e}", flush=True)
    assert e1 <= TOL and e2 <= TOL


def test_gemv_p5_decode_shape_vs_fp32():
    g = torch.Generator(device=DEV).manual_seed(5)
    N, K = 12288, 4096
    x = torch.randn(1, K, generator=g, device=DEV).to(torch.bfloat16)
    wg = (0.02 * torch.randn(N, K, generator=g, device=DEV)).to(torch.bfloat16)
    wu = (0.02 * torch.randn(N, K, generator=g, device=DEV)).to(torch.bfloat16)
    y = fused_ffn.gate_silu_mul_hip(x, wg.t(), wu.t())
    gf, uf = x.float() @ wg.float().t(), x.float() @ wu.float().t()
    ref = torch.nn.functional.silu(gf) * uf
    torch.cuda.synchronize()
    e1, e2 = max_rel_err(y, ref), rel_err(y, ref)
    print(f"gemv P5 decode: max_rel {e1:.2e} rel {e2:.2e}", flush=True)
    assert e1 <= TOL and e2 <= TOL


@pytest.mark.parametrize("M", [1, 5])
def test_linear_multi_equals_single_linears(M):
    """umic_linear_multi_bf16 over q/k/v-shaped linears (N 4096, 1024, 1024;
    a bias on one of them) equals umic_linear_bf16 on each, bit for bit, and
    the oracle to one ulp almost everywhere."""
    g = torch.Generator().manual_seed(90 + M)
    K = 1024
    x = bf16_randn(M, K, gen=g).to(DEV)
    ws = [bf16_randn(N, K, scale=0.05, gen=g).to(DEV) for N in (4096, 1024, 1024)]
    bs = [None, bf16_randn(1024, scale=0.5, gen=g).to(DEV), None]
    outs = linear.linear_multi_hip(x, ws, bs)
    singles = [linear.linear_hip(x, w, b) for w, b in zip(ws, bs)]
    torch.cuda.synchronize()
    for o, r, w, b in zip(outs, singles, ws, bs):
        assert o.shape == r.shape and torch.equal(o, r)
        _check_vs_oracle(o, oracle.linear(bits(x), bits(w), None if b is None else bits(b), 0,
                                          fused=True))


def test_linear_multi_empty_segment_and_rows_bound():
    g = torch.Generator().manual_seed(99)
    x = bf16_randn(2, 256, gen=g).to(DEV)
    w0, w2 = bf16_randn(64, 256, gen=g).to(DEV), bf16_randn(32, 256, gen=g).to(DEV)
    empty = torch.empty(0, 256, dtype=torch.bfloat16, device=DEV)
    o0, o1, o2 = linear.linear_multi_hip(x, [w0, empty, w2])
    torch.cuda.synchronize()
    assert o1.shape == (2, 0)
    assert torch.equal(o0, linear.linear_hip(x, w0)) and torch.equal(o2, linear.linear_hip(x, w2))
    with pytest.raises(ValueError):
        linear.linear_multi_hip(bf16_randn(9, 256, gen=g).to(DEV), [w0])


@pytest.mark.parametrize("M", [1, 8])
def test_linear_multi_single_segment(M):
    """One linear through the multi entry point (its operands come from the
    segment table, not the single-linear arguments) equals umic_linear_bf16."""
    g = torch.Generator().manual_seed(180 + M)
    x = bf16_randn(M, 256, gen=g).to(DEV)
    w = bf16_randn(64, 256, gen=g).to(DEV)
    (o,) = linear.linear_multi_hip(x, [w])
    ref = linear.linear_hip(x, w)
    torch.cuda.synchronize()
    assert torch.equal(o, ref)


@pytest.mark.parametrize("M,with_bias", [(1, False), (4, True)])
def test_linear_add_equals_linear_then_add(M, with_bias):
    """umic_linear_add_bf16 = the eager chain residual + linear(x): the same
    GEMV result rounded to bf16, then the bf16 sum, bit for bit."""
    g = torch.Generator().manual_seed(120 + M)
    N, K = 4096, 1536
    x = bf16_randn(1, M, K, gen=g).to(DEV)
    w = bf16_randn(N, K, scale=0.05, gen=g).to(DEV)
    b = bf16_randn(N, scale=0.5, gen=g).to(DEV) if with_bias else None
    r = bf16_randn(1, M, N, scale=4.0, gen=g).to(DEV)
    out = linear.linear_add_hip(x, w, b, r)
    ref = r + linear.linear_hip(x, w, b)
    torch.cuda.synchronize()
    assert out.shape == r.shape and torch.equal(out, ref)
