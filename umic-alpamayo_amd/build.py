"""Build libumic_hip.so (gfx950) from csrc/ with hipcc.

    python umic-alpamayo_amd/build.py        # incremental (object timestamps)
    python umic-alpamayo_amd/build.py --force

Each csrc/*.hip file compiles to its own object under _build/ (in parallel),
then all objects link into umic/lib/libumic_hip.so, the in-tree library the
umic package loads.  Flags: -O3, gfx950 only, no fp contraction (every fp32
rounding step in the kernels is explicit), and packed-fp32 codegen disabled.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(HERE, "umic", "lib")
LIB = os.path.join(LIB_DIR, "libumic_hip.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _deps() -> list[str]:
    hdrs = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hpp", ".h"))]
    hdrs += [os.path.join(INCLUDE, f) for f in os.listdir(INCLUDE) if f.endswith(".h")]
    return hdrs


def _compile(src: str, force: bool) -> str:
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    newest = max(os.path.getmtime(p) for p in [src, *_deps()])
    if force or not os.path.exists(obj) or os.path.getmtime(obj) < newest:
        cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        msgs = [ln for ln in (proc.stderr or "").splitlines()
                if "packed-fp32-ops' is not a recognized feature" not in ln]
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n" + "\n".join(msgs))
        if msgs:
            sys.stderr.write("\n".join(msgs) + "\n")
    return obj


def build(force: bool = False, jobs: int | None = None) -> str:
    """Compile every csrc/*.hip for gfx950 and link libumic_hip.so."""
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = _sources()
    with cf.ThreadPoolExecutor(max_workers=jobs or min(len(srcs), 8)) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    args = ap.parse_args()
    print(build(force=args.force))
