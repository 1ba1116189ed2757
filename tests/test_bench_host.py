"""bench.py's host-side traffic arithmetic (CPU): picking the calibration
copy and the kernel out of rocprofv3 counter-collection rows, and scaling
FETCH_SIZE / WRITE_SIZE by what they read for a copy of known size."""

from __future__ import annotations

import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402

P5 = "void umic::(anonymous namespace)::gemm_w4_kernel<2, 0, false>(umic::GemmArgs)"
COPY = "__amd_rocclr_copyBuffer"


def rows(*pairs):
    return [{"Kernel_Name": k, "Counter_Value": str(v)} for k, v in pairs]


def test_copy_and_kernel_take_the_last_dispatch_of_each():
    r = rows(("void at::native::fill_kernel", 5.0), (COPY, 100.0), (COPY, 262144.0),
             (P5, 1.0), ("void umic::gemm_w4_kernel<1, 0, false>", 7.0), (P5, 599641.875))
    assert bench.pmc_copy_and_kernel(r, bench.TRAFFIC_KERNELS["gate_silu_mul"]) == \
        (262144.0, 599641.875)


@pytest.mark.parametrize("r", [rows((P5, 1.0)), rows((COPY, 2.0)), rows((COPY, 0.0), (P5, 1.0))])
def test_missing_or_empty_calibration_is_reported(r):
    assert bench.pmc_copy_and_kernel(r, "gemm_w4_kernel<2,") is None


def test_counters_are_scaled_by_the_copy():
    kb = bench.COPY_BYTES / 1024
    # FETCH_SIZE reads half the copy's true bytes (scale 2), WRITE_SIZE all of them
    nbytes, info = bench.calibrated_traffic((kb / 2, 1000.0), (kb, 500.0))
    assert nbytes == (2 * 1000 + 500) * 1024
    assert info["read_scale"] == 2.0 and info["write_scale"] == 1.0
    assert info["fetch_kb"] == 1000.0 and info["write_kb"] == 500.0
