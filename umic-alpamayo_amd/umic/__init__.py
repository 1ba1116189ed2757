"""UMIC on MI355X: fused hot-path kernels for Qwen3-VL-family models.

Measurement-guided fusion layer with the reference's API (soonhong99/
umic-alpamayo, src/umic/__init__.py): no checkpoint modification, no
quantisation -- weights are shared and only the execution schedule of the
same math changes.  The fused path is hand-written gfx950 HIP (MFMA GEMMs,
single-pass norm and RoPE kernels) in libumic_hip.so, called through a C ABI.

Entry point:

    import umic
    report = umic.apply(model)   # patch all adopted fusions in place
"""

from umic.optimize import UmicConfig, apply

__all__ = ["apply", "UmicConfig"]
__version__ = "0.1.0"
