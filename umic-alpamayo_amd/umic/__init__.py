"""umic: the UMIC hot path of Alpamayo-family models on MI355X (gfx950).

``umic.apply(model)`` patches the fused kernels into a loaded model in place
and returns a report of what it matched; ``umic.UmicConfig`` selects the
fusions.  Weights are read where they are (nothing is converted or
quantised), and every fused site computes what the eager module computes:
bit for bit for the norms and RoPE, within GEMM rounding for the
projections.  The kernels are hand-written HIP in libumic_hip.so behind a C
ABI (include/umic_hip.h); the Python API is the reference package's
(soonhong99/umic-alpamayo, src/umic/__init__.py).
"""

from umic.optimize import UmicConfig, apply

__all__ = ["UmicConfig", "apply"]
__version__ = "0.1.0"
