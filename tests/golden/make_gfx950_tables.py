"""Write tests/golden/gfx950_rcp_rsq.npz: the gfx950 reciprocal and
reciprocal-square-root instructions as deltas from the correctly rounded
value, for the CPU oracle's restatement of torch-ROCm's LayerNorm.

torch-ROCm's bf16 LayerNorm (aten vectorized_layer_norm_kernel, block 64x4)
takes every Welford count reciprocal with v_rcp_f32 and the row's rstd with
v_rsq_f32 (fitted against its own mean/rstd outputs, see
tests/golden/make_eager_gpu.py).  Both instructions are approximations
(v_rcp_f32 differs from 1/n on ~10% of integers, v_rsq_f32 from 1/sqrt(x) on
~11% of [1, 4)), so the oracle reproduces them from these measured tables:

  rcp_delta[n-1]  bits(v_rcp_f32(n)) - bits((float)(1.0 / n)),  n = 1..65536
  rsq_delta2      v_rsq_f32(x) - (float)(1.0 / sqrt((double)x)) in ulps for
                  every float x of [1, 4), packed 2 bits per value
                  (code = delta + 1; deltas are -1, 0 or +1)

Both instructions scale exactly with the exponent (rsq(x * 4^k) =
rsq(x) * 2^-k, rcp(x * 2^k) = rcp(x) * 2^-k, checked on the device over
1M samples x 81 scales), so [1, 4) covers every normal input.  Run on a
gfx950 box (builds gfx950_tables.hip with hipcc):

    python tests/golden/make_gfx950_tables.py [OUT.npz]
"""

from __future__ import annotations

import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "gfx950_rcp_rsq.npz")


def main(out: str = OUT) -> None:
    with tempfile.TemporaryDirectory() as tmp:
        exe = os.path.join(tmp, "gfx950_tables")
        subprocess.run(["hipcc", "--offload-arch=gfx950", "-O2", "-Xclang", "-target-feature",
                        "-Xclang", "-packed-fp32-ops", os.path.join(HERE, "gfx950_tables.hip"),
                        "-o", exe], check=True)
        rcp_p, rsq_p = os.path.join(tmp, "rcp.bin"), os.path.join(tmp, "rsq.bin")
        subprocess.run([exe, rcp_p, rsq_p], check=True, timeout=120)
        rcp = np.fromfile(rcp_p, dtype=np.float32)
        rsq = np.fromfile(rsq_p, dtype=np.float32)
    n = np.arange(1, rcp.size + 1, dtype=np.float64)
    rcp_cr = (1.0 / n).astype(np.float32)
    rcp_delta = rcp.view(np.int32).astype(np.int64) - rcp_cr.view(np.int32)
    x = (np.arange(rsq.size, dtype=np.int64) + 0x3F800000).astype(np.uint32).view(np.float32)
    rsq_cr = (1.0 / np.sqrt(x.astype(np.float64))).astype(np.float32)
    rsq_delta = rsq.view(np.int32).astype(np.int64) - rsq_cr.view(np.int32)
    assert np.abs(rcp_delta).max() <= 1 and np.abs(rsq_delta).max() <= 1
    code = (rsq_delta + 1).astype(np.uint8)
    packed = code[0::4] | (code[1::4] << 2) | (code[2::4] << 4) | (code[3::4] << 6)
    np.savez_compressed(out, rcp_delta=rcp_delta.astype(np.int8), rsq_delta2=packed)
    print(f"wrote {out}: rcp {int((rcp_delta != 0).sum())} of {rcp.size} off CR, "
          f"rsq {int((rsq_delta != 0).sum())} of {rsq.size} off CR")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else OUT)
