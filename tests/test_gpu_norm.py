"""GPU parity: RMSNorm / add+RMSNorm / LayerNorm / add+LayerNorm kernels.

Each case draws seeded inputs on the CPU (fp32 -> bf16, identical bits on both
sides), runs the HIP kernel through the C ABI (umic.kernels wrappers) and
compares with the CPU oracle bit for bit, including the BASELINE shapes
[3100, 4096] (RMSNorm), [99200, 128] (q_norm rows) and [16384, 1280] (ViT LN),
and every launch regime of the row statistic (register paths, the decode
rows, the row split at n >= 8192, scalar rows below n = 128, LayerNorm rows
off 8-byte alignment).  At the BASELINE and decode shapes the kernel is also
compared with torch eager (the transformers modules) on the same GPU: within
one bf16 ulp -- the bar -- and, since the kernels reproduce eager's fp32
reduction order, identical; the ulp histograms go to $UMIC_PARITY_LOG.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from helpers import bf16_randn, bits, log_parity, ulp, ulp_hist

import oracle
from umic.kernels import layernorm, rmsnorm

pytestmark = pytest.mark.gpu
DEV = "cuda"

# (rows, n): BASELINE shapes, decode row, empty, q/k_norm rows, ragged lane
# tails (n=1000, 80), rows beyond the register path (n=8200, 16384) and
# n % 8 != 0 (generic kernel).  Rows of one or two vectors per lane take 4 or
# 2 rows per lane group from 16384 rows up: (99200, 128) and (24800, 128) do,
# (16390, 128) and (16387, 1024) with a ragged last group, (64, 128) does not.
RMS_SHAPES = [(3100, 4096), (257, 4096), (1, 4096), (0, 4096), (99200, 128), (24800, 128),
              (16390, 128), (16387, 1024), (64, 128),
              (333, 1280), (64, 1000), (77, 80), (9, 8200), (5, 16384), (31, 100), (3, 2)]
LN_SHAPES = [(16384, 1280), (4096, 1152), (100, 4096), (1, 1280), (0, 1280), (64, 1000),
             (16390, 128), (16387, 1024), (50, 80), (7, 8200), (13, 100)]


def _inputs(rows, n, seed):
    g = torch.Generator().manual_seed(seed)
    x = bf16_randn(rows, n, gen=g)
    r = bf16_randn(rows, n, gen=g)
    w = bf16_randn(n, scale=0.1, shift=1.0, gen=g)
    b = bf16_randn(n, scale=0.1, gen=g)
    return x, r, w, b


@pytest.mark.parametrize("rows,n", RMS_SHAPES)
def test_rmsnorm_matches_oracle(rows, n):
    x, r, w, _ = _inputs(rows, n, seed=rows * 7 + n)
    y = rmsnorm.rmsnorm_hip(x.to(DEV), w.to(DEV), 1e-6)
    torch.cuda.synchronize()
    assert y.shape == x.shape and y.dtype == torch.bfloat16
    assert np.array_equal(bits(y), oracle.rmsnorm(bits(x), bits(w), 1e-6))


@pytest.mark.parametrize("rows,n", RMS_SHAPES)
def test_add_rmsnorm_matches_oracle(rows, n):
    x, r, w, _ = _inputs(rows, n, seed=rows * 11 + n)
    normed, summed = rmsnorm.add_rmsnorm_hip(x.to(DEV), r.to(DEV), w.to(DEV), 1e-6)
    torch.cuda.synchronize()
    on, os_ = oracle.add_rmsnorm(bits(x), bits(r), bits(w), 1e-6)
    assert np.array_equal(bits(summed), os_)
    assert np.array_equal(bits(normed), on)


@pytest.mark.parametrize("rows,n", LN_SHAPES)
def test_layernorm_matches_oracle(rows, n):
    x, r, w, b = _inputs(rows, n, seed=rows * 13 + n)
    y = layernorm.layernorm_hip(x.to(DEV), w.to(DEV), b.to(DEV), 1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(bits(y), oracle.layernorm(bits(x), bits(w), bits(b), 1e-6))


@pytest.mark.parametrize("rows,n", LN_SHAPES)
def test_add_layernorm_matches_oracle(rows, n):
    x, r, w, b = _inputs(rows, n, seed=rows * 17 + n)
    normed, summed = layernorm.add_layernorm_hip(x.to(DEV), r.to(DEV), w.to(DEV), b.to(DEV),
                                                 1e-6)
    torch.cuda.synchronize()
    on, os_ = oracle.add_layernorm(bits(x), bits(r), bits(w), bits(b), 1e-6)
    assert np.array_equal(bits(summed), os_)
    assert np.array_equal(bits(normed), on)


def test_strided_and_misaligned_rows():
    """Row stride > n (a column slice) takes the vector kernel with ldx;
    a base pointer off 16-byte alignment takes the generic kernel."""
    g = torch.Generator().manual_seed(5)
    big = bf16_randn(300, 4160, gen=g)
    w = bf16_randn(4096, scale=0.1, shift=1.0, gen=g)
    xs = big[:, :4096]
    y = rmsnorm.rmsnorm_hip(big.to(DEV)[:, :4096], w.to(DEV), 1e-6)
    assert np.array_equal(bits(y), oracle.rmsnorm(bits(xs), bits(w), 1e-6))
    flat = bf16_randn(1 + 200 * 1280, gen=g)
    xm = flat[1:].view(200, 1280)
    wl, bl = bf16_randn(1280, gen=g), bf16_randn(1280, gen=g)
    dm = flat.to(DEV)[1:].view(200, 1280)
    assert dm.data_ptr() % 16 != 0
    y = layernorm.layernorm_hip(dm, wl.to(DEV), bl.to(DEV), 1e-5)
    # eager's layer_norm takes its scalar row-moments kernel for such a base;
    # the library follows that kernel's order, as the oracle does with aligned=False
    assert np.array_equal(bits(y), oracle.layernorm(bits(xm), bits(wl), bits(bl), 1e-5,
                                                    aligned=False))


def test_leading_dims_and_eps():
    g = torch.Generator().manual_seed(6)
    x = bf16_randn(2, 3, 50, 128, gen=g)
    w = bf16_randn(128, scale=0.1, shift=1.0, gen=g)
    for eps in (1e-6, 1e-5, 0.5):
        y = rmsnorm.rmsnorm_hip(x.to(DEV), w.to(DEV), eps)
        assert y.shape == x.shape
        assert np.array_equal(bits(y).reshape(-1, 128),
                              oracle.rmsnorm(bits(x).reshape(-1, 128), bits(w), eps))


def _hf_rms(x, w, eps=1e-6):
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextRMSNorm

    m = Qwen3VLTextRMSNorm(x.shape[-1], eps=eps).to(device=x.device, dtype=torch.bfloat16)
    with torch.no_grad():
        m.weight.copy_(w)
        return m(x)


# (op, eager-layout shape): the BASELINE config 2 / 5 norms in the layouts HF
# calls them with -- LM rows [1, 3100, 4096], the q_norm / k_norm head rows
# [1, 3100, H, 128] (99200 / 24800 rows), the decode rows ([1, 1, 4096] and
# 32 / 8 head rows), the ViT rows [16384, 1280] -- a SigLIP-width LN, and
# batched decode rows (1 to 7 rows of 512 .. 4096).
EAGER_CASES = [("rmsnorm", (1, 3100, 4096)), ("add_rmsnorm", (1, 3100, 4096)),
               ("rmsnorm", (1, 3100, 32, 128)), ("rmsnorm", (1, 3100, 8, 128)),
               ("rmsnorm", (1, 1, 4096)), ("add_rmsnorm", (1, 1, 4096)),
               ("rmsnorm", (1, 1, 32, 128)), ("rmsnorm", (1, 1, 8, 128)),
               ("layernorm", (16384, 1280)), ("add_layernorm", (16384, 1280)),
               ("layernorm", (4096, 1152)),
               # one to seven rows: 128 .. 512 reducing threads per row
               ("rmsnorm", (2, 4096)), ("add_rmsnorm", (3, 4096)), ("rmsnorm", (5, 4096)),
               ("add_rmsnorm", (7, 4096)), ("rmsnorm", (1, 1280)), ("rmsnorm", (3, 1152)),
               ("add_rmsnorm", (1, 2048)), ("rmsnorm", (6, 512))]


@pytest.mark.parametrize("op,shape", EAGER_CASES)
def test_norm_vs_torch_eager_on_gpu(op, shape):
    """The kernel against the eager module on the same GPU and inputs: at
    most one bf16 ulp apart (the bar), and identical."""
    print(f"eager parity {op} {shape}", flush=True)
    n = shape[-1]
    g = torch.Generator().manual_seed(len(shape) * 1000 + n + shape[-2])
    x = bf16_randn(*shape, gen=g).to(DEV)
    r = bf16_randn(*shape, gen=g).to(DEV)
    w = bf16_randn(n, scale=0.1, shift=1.0, gen=g).to(DEV)
    b = bf16_randn(n, scale=0.1, gen=g).to(DEV)
    with torch.no_grad():
        if op == "rmsnorm":
            got, ref = rmsnorm.rmsnorm_hip(x, w, 1e-6), _hf_rms(x, w)
        elif op == "add_rmsnorm":
            got, summed = rmsnorm.add_rmsnorm_hip(x, r, w, 1e-6)
            s_ref = r + x  # the decoder layer's `residual + hidden_states`
            assert torch.equal(summed, s_ref)
            ref = _hf_rms(s_ref, w)
        elif op == "layernorm":
            got = layernorm.layernorm_hip(x, w, b, 1e-6)
            ref = torch.nn.functional.layer_norm(x, (n,), w, b, 1e-6)
        else:
            got, summed = layernorm.add_layernorm_hip(x, r, w, b, 1e-6)
            s_ref = r + x
            assert torch.equal(summed, s_ref)
            ref = torch.nn.functional.layer_norm(s_ref, (n,), w, b, 1e-6)
    torch.cuda.synchronize()
    d = ulp(bits(got), bits(ref))
    log_parity(op, shape, d)
    assert d.max() <= 1, ulp_hist(d)
    assert (d == 0).all(), ulp_hist(d)
