"""GPU: the norm kernels against torch eager on the same GPU over a seeded
sweep of shapes that crosses every launch regime of torch's reductions.

RMSNorm follows aten's reduction plan for its width and row count (vector or
scalar loads, 1..512 reducing threads per row, split rows) and must be bit
for bit eager's HF Qwen3VLTextRMSNorm chain, also for widths that are not a
multiple of 4 and for rows that start off 16-byte alignment.  LayerNorm
follows eager's vectorized kernel where eager takes it (width a multiple of
4, 8-byte aligned input) and its scalar row-moments kernel elsewhere: bit
for bit in both.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from helpers import bf16_randn, bits, log_parity, ulp

from umic.kernels import layernorm, rmsnorm

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _shapes(seed: int, count: int):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        rows = int(rng.choice([1, 2, 3, 5, 7, 8, 13, 64, 100, 257, 1000, 4999]))
        n = int(rng.choice([4, 12, 80, 100, 127, 128, 130, 256, 510, 512, 1000, 1152, 1280,
                            2048, 3000, 4096, 5120, 8192]))
        out.append((rows, n))
    return out


SHAPES = _shapes(2024, 36)


def _hf_rms(x, w, eps=1e-6):
    var = x.float().pow(2).mean(-1, keepdim=True)
    return w * (x.float() * torch.rsqrt(var + eps)).to(x.dtype)


@pytest.mark.parametrize("rows,n", SHAPES)
def test_rmsnorm_sweep_vs_eager(rows, n):
    print(f"rms sweep rows={rows} n={n}", flush=True)
    g = torch.Generator().manual_seed(rows * 10007 + n)
    x = bf16_randn(rows, n, gen=g).to(DEV)
    r = bf16_randn(rows, n, gen=g).to(DEV)
    w = bf16_randn(n, scale=0.1, shift=1.0, gen=g).to(DEV)
    with torch.no_grad():
        got = rmsnorm.rmsnorm_hip(x, w, 1e-6)
        ref = _hf_rms(x, w)
        normed, summed = rmsnorm.add_rmsnorm_hip(x, r, w, 1e-6)
        s_ref = r + x
        ref2 = _hf_rms(s_ref, w)
    torch.cuda.synchronize()
    assert torch.equal(summed, s_ref)
    for name, a, b in (("rmsnorm", got, ref), ("add_rmsnorm", normed, ref2)):
        d = ulp(bits(a), bits(b))
        log_parity(f"{name} sweep", (rows, n), d)
        assert (d == 0).all(), (name, int(d.max()), int((d > 0).sum()))


@pytest.mark.parametrize("rows,n", SHAPES[:18])
def test_rmsnorm_sweep_offset_rows(rows, n):
    """Rows that start 2 bytes past 16-byte alignment (a view one element
    into a wider buffer): eager's reduction then reads its fp32 copy with a
    per-row head and tail; the kernel follows it."""
    g = torch.Generator().manual_seed(rows * 7919 + n)
    big = bf16_randn(rows, n + 1, gen=g).to(DEV)
    x = big[:, 1:]
    w = bf16_randn(n, scale=0.1, shift=1.0, gen=g).to(DEV)
    with torch.no_grad():
        got = rmsnorm.rmsnorm_hip(x, w, 1e-6)
        ref = _hf_rms(x, w)
    torch.cuda.synchronize()
    d = ulp(bits(got), bits(ref))
    assert (d == 0).all(), (int(d.max()), int((d > 0).sum()))


@pytest.mark.parametrize("rows,n", SHAPES)
def test_layernorm_sweep_vs_eager(rows, n):
    print(f"ln sweep rows={rows} n={n}", flush=True)
    g = torch.Generator().manual_seed(rows * 10009 + n)
    x = bf16_randn(rows, n, gen=g).to(DEV)
    r = bf16_randn(rows, n, gen=g).to(DEV)
    w = bf16_randn(n, scale=0.1, shift=1.0, gen=g).to(DEV)
    b = bf16_randn(n, scale=0.1, gen=g).to(DEV)
    with torch.no_grad():
        got = layernorm.layernorm_hip(x, w, b, 1e-6)
        ref = torch.nn.functional.layer_norm(x, (n,), w, b, 1e-6)
        normed, summed = layernorm.add_layernorm_hip(x, r, w, b, 1e-6)
        s_ref = r + x
        ref2 = torch.nn.functional.layer_norm(s_ref, (n,), w, b, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(summed, s_ref)
    for name, a, bb in (("layernorm", got, ref), ("add_layernorm", normed, ref2)):
        d = ulp(bits(a), bits(bb))
        log_parity(f"{name} sweep", (rows, n), d)
        assert (d == 0).all(), (name, int(d.max()), int((d > 0).sum()))


@pytest.mark.parametrize("rows,n", [(r, n) for r, n in SHAPES if n % 4 == 0][:10])
def test_layernorm_sweep_offset_rows(rows, n):
    """x read 2 bytes past 8-byte alignment: eager takes its scalar kernel
    for a width that is a multiple of 4 too; the library follows it."""
    g = torch.Generator().manual_seed(rows * 7907 + n)
    flat = bf16_randn(rows * n + 1, gen=g).to(DEV)
    x = flat[1:].view(rows, n)
    w = bf16_randn(n, scale=0.1, shift=1.0, gen=g).to(DEV)
    b = bf16_randn(n, scale=0.1, gen=g).to(DEV)
    with torch.no_grad():
        got = layernorm.layernorm_hip(x, w, b, 1e-6)
        ref = torch.nn.functional.layer_norm(x, (n,), w, b, 1e-6)
    torch.cuda.synchronize()
    d = ulp(bits(got), bits(ref))
    log_parity("layernorm offset sweep", (rows, n), d)
    assert (d == 0).all(), (int(d.max()), int((d > 0).sum()))
