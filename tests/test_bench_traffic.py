"""bench.py's HBM-traffic arithmetic (no GPU): counter means from rocprofv3 counter rows and
their scaling by a copy of known size."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def _row(kernel, counter, value):
    return {"Kernel_Name": kernel, "Counter_Name": counter, "Counter_Value": str(value)}


def test_counter_means_split_copy_and_other_kernels():
    # two attention dispatches, the three copies split over four dispatches, unrelated kernels
    # and another counter in the same file
    rows = [_row("void tree_attn_bf16_kernel<8>(AttnArgs, int)", "FETCH_SIZE", 100.0),
            _row("void tree_attn_bf16_kernel<8>(AttnArgs, int)", "FETCH_SIZE", 300.0),
            _row("__amd_rocclr_copyBuffer", "FETCH_SIZE", 98316.0),
            _row("__amd_rocclr_copyBuffer", "FETCH_SIZE", 98316.0),
            _row("__amd_rocclr_copyBuffer", "FETCH_SIZE", 98316.0),
            _row("__amd_rocclr_copyBuffer", "FETCH_SIZE", 98316.0),
            _row("at::native::fill_kernel", "FETCH_SIZE", 7.0),
            _row("void tree_attn_bf16_kernel<8>(AttnArgs, int)", "WRITE_SIZE", 5.0)]
    got = bench.counter_means(rows, "FETCH_SIZE", "tree_attn_bf16_kernel")
    assert got == (200.0, 4 * 98316.0 / bench.COPY_REPS)
    assert bench.counter_means(rows, "WRITE_SIZE", "tree_attn_bf16_kernel") is None  # no copy rows


def test_traffic_scales_each_counter_by_its_copy():
    copy_kib = bench.COPY_BYTES / 1024.0
    # FETCH_SIZE counts half the copy's bytes, WRITE_SIZE all of them
    means = {"FETCH_SIZE": (1000.0, copy_kib / 2), "WRITE_SIZE": (10.0, copy_kib)}
    total, detail = bench.traffic_from_means(means)
    assert total == int(1000.0 * 1024 * 2 + 10.0 * 1024)
    assert detail["FETCH_SIZE"]["scale"] == 2.0 and detail["WRITE_SIZE"]["scale"] == 1.0
