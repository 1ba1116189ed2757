"""CPU: no compiler-made accumulator read between an MFMA and its fence.

The four-wave GEMM core issues its MFMAs as inline asm (tied "+a" AGPR
accumulators), which the compiler's hazard checks do not see into: reading
an accumulator too soon after the MFMA that writes it returns a stale value.
The kernels read results only after fence_results() (four `s_nop 7` in
statements that take every accumulator), so in the compiled code no
instruction between an MFMA and the next `s_nop 7` may name an AGPR -- a
register-allocator copy or spill there is exactly the hazard.  This builds
csrc/gemm.hip to gfx950 assembly with the library's flags and scans every
kernel in text order (a superset of the control-flow paths).
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "umic-alpamayo_amd")

AGPR = re.compile(r"\ba\[\d+:\d+\]|\ba\d+\b")


def agpr_reads_before_fence(asm: str) -> dict[str, list[tuple[int, str]]]:
    """{kernel: [(line, instruction)]} of AGPR-naming instructions that
    follow an MFMA before the next `s_nop 7`, in text order."""
    bad: dict[str, list[tuple[int, str]]] = {}
    fn, armed = None, False
    for i, line in enumerate(asm.splitlines(), 1):
        s = line.strip()
        m = re.match(r"^(_Z\S+):", s)
        if m:
            fn, armed = m.group(1), False
            continue
        if not s or s.startswith((";", ".")):
            continue
        if s.startswith("v_mfma"):
            armed = True
            continue
        if s.startswith("s_nop 7"):
            armed = False
            continue
        if armed and AGPR.search(s.split(";")[0]):
            bad.setdefault(fn, []).append((i, s))
    return bad


def test_scanner_flags_a_read_after_an_mfma():
    asm = "\n".join(["_ZN4umic1kEv:", "v_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[4:7], a[0:3]",
                     "v_accvgpr_read_b32 v8, a3", "s_nop 7", "v_accvgpr_read_b32 v9, a2"])
    assert agpr_reads_before_fence(asm) == {"_ZN4umic1kEv": [(3, "v_accvgpr_read_b32 v8, a3")]}


@pytest.mark.skipif(shutil.which(os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")) is None,
                    reason="hipcc not installed")
def test_gemm_kernels_read_accumulators_only_after_the_fence(tmp_path):
    sys.path.insert(0, PKG)
    import build

    src = os.path.join(PKG, "csrc", "gemm.hip")
    out = tmp_path / "gemm.s"
    cmd = [build.HIPCC, *build.CFLAGS, f"-I{build.INCLUDE}", "-S", "--cuda-device-only", src,
           "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    asm = out.read_text()
    assert asm.count("v_mfma") > 1000  # the four-wave core's instantiations are there
    bad = agpr_reads_before_fence(asm)
    assert not bad, {k[:80]: v[:4] for k, v in bad.items()}
