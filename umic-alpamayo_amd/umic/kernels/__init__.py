"""Kernel registry: fused-pattern name -> implementation.

Same surface as the reference's registry (src/umic/kernels/__init__.py:14-23),
pre-populated with this runtime's gfx950 kernels.  Every wrapper here runs
the HIP library and raises if it is missing; eager fallbacks for ineligible
inputs are applied by umic.integrate, never inside a kernel wrapper.
"""

from __future__ import annotations

import logging
from typing import Callable

logger = logging.getLogger(__name__)

_KERNELS: dict[str, Callable] = {}


def register_kernel(pattern_name: str, fn: Callable) -> None:
    _KERNELS[pattern_name] = fn
    logger.info("kernel registered: %s -> %s", pattern_name, fn.__name__)


def get_kernel(pattern_name: str) -> Callable | None:
    return _KERNELS.get(pattern_name)


def _register_builtin() -> None:
    from umic.kernels import fused_ffn, layernorm, linear, rmsnorm, rope

    for name, fn in (
        ("gate_silu_mul", fused_ffn.gate_silu_mul_hip),
        ("linear", linear.linear_hip),
        ("rmsnorm", rmsnorm.rmsnorm_hip),
        ("add_rmsnorm", rmsnorm.add_rmsnorm_hip),
        ("layernorm", layernorm.layernorm_hip),
        ("add_layernorm", layernorm.add_layernorm_hip),
        ("rope_text", rope.apply_rotary_text_hip),
        ("rope_vision", rope.apply_rotary_vision_hip),
    ):
        _KERNELS[name] = fn


_register_builtin()
