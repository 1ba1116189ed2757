"""CPU: no compiler-made accumulator read between an MFMA and its fence, and
no early overwrite of an inline-asm store's data registers.

The four-wave GEMM core issues its MFMAs as inline asm (tied "+a" AGPR
accumulators), which the compiler's hazard checks do not see into: reading
an accumulator too soon after the MFMA that writes it returns a stale value.
The kernels read results only after fence_results() (four `s_nop 7`, then
statements that take each live accumulator), so in the compiled code no
instruction between an MFMA and the next `s_nop 7` may name an AGPR -- a
register-allocator copy or spill there is exactly the hazard.  The stream-K
partial stores are inline asm too: a store of more than 8 bytes reads its
data registers after issue, so the next two wait states may not write them
(the asm spaces each store with `s_nop 1`; a copy of the next block into the
same registers right after the store gave run-to-run different partials).
This builds csrc/gemm.hip to gfx950 assembly with the library's flags and
scans every kernel in text order (a superset of the control-flow paths).
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


VREG = re.compile(r"^v(\d+)$|^v\[(\d+):(\d+)\]$")


def _vrange(tok: str):
    m = VREG.match(tok.strip())
    if not m:
        return None
    if m.group(1) is not None:
        return int(m.group(1)), int(m.group(1))
    return int(m.group(2)), int(m.group(3))


def store_data_overwrites(asm: str, wait_states: int = 2) -> list[tuple[int, str]]:
    """[(line, instruction)] of VALU writes to the data registers of an
    inline-asm store of more than 8 bytes within `wait_states` wait states of
    it.  Such a store reads its data after issue, and the compiler's hazard
    checks (which space its own stores) do not see into inline asm; gfx950
    needs two wait states (an `s_nop N` counts N + 1)."""
    bad = []
    in_asm = False
    pending = None  # (first, last, wait states left)
    for i, line in enumerate(asm.splitlines(), 1):
        s = line.strip()
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not s or s.startswith((";", ".")) or s.endswith(":"):
            continue
        op, _, rest = s.split(";")[0].partition(" ")
        args = [a.strip() for a in rest.split(",")]
        if pending is not None:
            lo, hi, left = pending
            if op == "s_nop":
                left -= int(args[0], 0) + 1
            else:
                r = _vrange(args[0]) if op.startswith("v_") and args else None
                if r and r[0] <= hi and lo <= r[1]:
                    bad.append((i, s))
                left -= 1
            pending = (lo, hi, left) if left > 0 else None
        if in_asm and re.match(r"^(global|buffer|flat)_store_dwordx[34]$", op):
            data = args[1] if op.startswith(("global", "flat")) else args[0]
            r = _vrange(data)
            if r:
                pending = (r[0], r[1], wait_states)
    return bad


def test_store_scanner_flags_an_early_overwrite():
    asm = "\n".join([";;#ASMSTART", "global_store_dwordx4 v[8:9], v[0:3], off sc1", ";;#ASMEND",
                     "v_accvgpr_read_b32 v0, a4"])
    assert store_data_overwrites(asm) == [(4, "v_accvgpr_read_b32 v0, a4")]
    spaced = asm.replace("off sc1", "off sc1\n\ts_nop 1")
    assert store_data_overwrites(spaced) == []


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
    assert asm.count("global_store_dwordx4") > 0
    early = store_data_overwrites(asm)
    assert not early, early[:4]
