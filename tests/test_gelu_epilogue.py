"""CPU: the linear's GELU epilogues (csrc/gemm.hip gelu_erf, gelu_tanh).

The kernel takes erf(|u|) = 1 - erfc(|u|) with erfc(z) = t * exp(-z^2 + P(t)),
t = 1/(1 + z/2) and fitted coefficients for P, then forms GELU exactly as eager
does, 0.5 * x * (1 + erf(x / sqrt2)) in fp32.  This test reads the coefficients
from the kernel source, evaluates the formula in float32 as the kernel does
(fma Horner steps, float32 products), and checks it against scipy in float64:
erfc to 1.5e-5 relative on [0, 9] (below that, fp32 subnormals), erf to 4e-7
absolute, and the bf16 GELU against eager's fp32 chain built on a correctly
rounded erf (the oracle's glibc erff) to one ulp, identical almost everywhere
-- so a mistyped or reordered coefficient fails here.  The tanh form,
tanh|y| = 1 - 2 / (1 + exp(2|y|)), is checked the same way against a correctly
rounded tanh, and against torch's own gelu(approximate="tanh").  The GPU
parity tests then compare the fused linear's GELU outputs with the oracle.
"""

from __future__ import annotations

import os
import re

import numpy as np
import torch
from scipy.special import erf, erfc

SRC = os.path.join(os.path.dirname(__file__), "..", "umic-alpamayo_amd", "csrc", "gemm.hip")
F32 = np.float32


def _coefficients() -> list[float]:
    text = open(SRC).read()
    body = text[text.index("float gelu_erf(float x)"):]
    body = body[:body.index("return")]
    first = re.search(r"float p = ([-+0-9.e]+)f;", body).group(1)
    rest = re.findall(r"__builtin_fmaf\(p, t, ([-+0-9.e]+)f\)", body)
    return [float(first)] + [float(c) for c in rest]   # highest degree first


def _erfc32(z: np.ndarray, coef: list[float]) -> np.ndarray:
    """The kernel's fp32 erfc (exp2 evaluated exactly: the hardware's ~1 ulp
    is within the margins below)."""
    z = z.astype(F32)
    t = (F32(1) / (F32(1) + F32(0.5) * z)).astype(F32)
    p = np.full_like(t, F32(coef[0]))
    for c in coef[1:]:
        p = (p.astype(np.float64) * t + F32(c)).astype(F32)    # one rounding: fma
    arg = ((p - (z * z).astype(F32)).astype(F32) * F32(1.4426950408889634)).astype(F32)
    return (t.astype(np.float64) * np.exp2(arg.astype(np.float64))).astype(F32)


def _gelu32(x: np.ndarray, coef: list[float]) -> np.ndarray:
    x = x.astype(F32)
    z = (np.abs(x) * F32(0.70710678118654752)).astype(F32)
    erf_abs = (F32(1) - _erfc32(z, coef)).astype(F32)
    one_plus = (F32(1) + np.where(x < 0, -erf_abs, erf_abs)).astype(F32)
    return (F32(0.5) * x * one_plus).astype(F32)


def test_coefficients_parse():
    assert len(_coefficients()) == 10


def test_erfc_relative_error_on_0_9():
    z = np.concatenate([np.linspace(0, 9, 400001), np.geomspace(1e-8, 1e-2, 2001)]).astype(F32)
    approx = _erfc32(z, _coefficients()).astype(np.float64)
    ref = erfc(z.astype(np.float64))
    assert (np.abs(approx - ref) / ref).max() < 1.5e-5


def test_erf_absolute_error():
    z = np.linspace(0, 8, 800001).astype(F32)
    mine = (F32(1) - _erfc32(z, _coefficients())).astype(np.float64)
    ref = erf(z.astype(np.float64))
    assert np.abs(mine - ref).max() <= 4e-7      # inside 1 + erf: ~3 fp32 ulps of 1


def test_gelu_matches_eager_fp32_chain_in_bf16():
    x = np.concatenate([np.linspace(-10, 10, 2000001), np.linspace(-0.01, 0.01, 20001)]).astype(F32)
    mine = torch.from_numpy(_gelu32(x, _coefficients())).to(torch.bfloat16)
    # eager's chain, 0.5 * x * (1 + erf(x / sqrt2)) in fp32, on a correctly
    # rounded erf (float64 erf rounded to fp32, as glibc's erff gives)
    u = (x * F32(0.70710678118654752)).astype(F32)
    erf32 = erf(u.astype(np.float64)).astype(F32)
    ref32 = (F32(0.5) * x * (F32(1) + erf32).astype(F32)).astype(F32)
    eager = torch.from_numpy(ref32).to(torch.bfloat16)
    a = mine.view(torch.int16).numpy().astype(np.int32)
    b = eager.view(torch.int16).numpy().astype(np.int32)
    # bf16 patterns of same-sign values: ulp distance = pattern difference
    same = (a == b)
    assert same.mean() > 0.999
    assert np.abs(a - b)[np.sign(a) == np.sign(b)].max() <= 1


def _tanh_constants() -> tuple[float, float, float]:
    text = open(SRC).read()
    body = text[text.index("float gelu_tanh(float x)"):]
    body = body[:body.index("return")]
    c, k = re.search(r"float y = ([0-9.e]+)f \* \(x \+ ([0-9.e]+)f \*", body).groups()
    l2 = re.search(r"__builtin_fabsf\(y\) \* ([0-9.e]+)f", body).group(1)
    return float(c), float(k), float(l2)


def _gelu_tanh32(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The kernel's fp32 steps (exp2 and the reciprocal correctly rounded: the
    hardware's ~1 ulp moves tanh|y| by far less than its fp32 grid near 1)."""
    c, k, l2 = (F32(v) for v in _tanh_constants())
    x = x.astype(F32)
    cube = (x * x * x).astype(F32)
    y = (c * (x + k * cube).astype(F32)).astype(F32)
    with np.errstate(over="ignore"):
        e = np.exp2((np.abs(y) * l2).astype(F32).astype(np.float64)).astype(F32)
    r = (1.0 / (F32(1) + e).astype(np.float64)).astype(F32)
    th_abs = (F32(1) - F32(2) * r).astype(F32)
    th = np.where(y < 0, -th_abs, th_abs).astype(F32)
    return (F32(0.5) * x * (F32(1) + th).astype(F32)).astype(F32), th


def test_tanh_constants():
    c, k, l2 = _tanh_constants()
    assert abs(c - np.sqrt(2 / np.pi)) < 1e-12
    assert k == 0.044715
    assert abs(l2 - 2 / np.log(2)) < 1e-12


def test_tanh_absolute_error():
    x = np.linspace(-12, 12, 1200001).astype(F32)
    _, th = _gelu_tanh32(x)
    c, k, _ = (F32(v) for v in _tanh_constants())
    y = (c * (x + k * (x * x * x).astype(F32)).astype(F32)).astype(F32)
    assert np.abs(th.astype(np.float64) - np.tanh(y.astype(np.float64))).max() <= 1.2e-7


def _bf16_bits(a: np.ndarray) -> np.ndarray:
    return torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().astype(np.int32)


def test_gelu_tanh_matches_eager_fp32_chain_in_bf16():
    x = np.concatenate([np.linspace(-12, 12, 2400001), np.linspace(-0.01, 0.01, 20001)]).astype(F32)
    mine, _ = _gelu_tanh32(x)
    # eager's chain in fp32 on a correctly rounded tanh
    cube = (x * x * x).astype(F32)
    y = (F32(0.7978845608028654) * (x + F32(0.044715) * cube).astype(F32)).astype(F32)
    tanh32 = np.tanh(y.astype(np.float64)).astype(F32)
    ref32 = (F32(0.5) * x * (F32(1) + tanh32).astype(F32)).astype(F32)
    a, b = _bf16_bits(mine), _bf16_bits(ref32)
    assert (a == b).mean() > 0.999
    assert np.abs(a - b)[np.sign(a) == np.sign(b)].max() <= 1
    # and torch's own CPU kernel of the same activation, above the negative
    # tail: its vectorised CPU tanh departs from tanh there (x in about
    # [-5.2, -3.5]), where the GPU's eager kernel uses the device tanhf
    t = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    c = _bf16_bits(t)
    keep = x > -3.4
    assert (a[keep] == c[keep]).mean() > 0.999
    assert np.abs(a - c)[keep & (np.sign(a) == np.sign(c))].max() <= 1
