"""The rocprofv3 CSV readers of aster_amd.profiling, on hand-made counter files."""

import csv
import os

import pytest

from aster_amd import profiling


def _counters(root, rows):
    os.makedirs(root, exist_ok=True)
    with open(os.path.join(root, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for name, counter, value in rows:
            w.writerow({"Kernel_Name": name, "Counter_Name": counter, "Counter_Value": value})


def test_summarize_median_and_names(tmp_path):
    k = "void (anonymous namespace)::decode_streamk_kernel<bf16_t, 128, 4, false>(AttnArgs)"
    _counters(tmp_path / "a", [(k, "FETCH_SIZE", v) for v in (10, 1000, 1002, 1004)] +
              [("other_kernel(int)", "FETCH_SIZE", 5)])
    table = profiling.summarize(str(tmp_path / "a"), "decode")
    assert list(table) == [("decode_streamk_kernel<bf16_t, 128, 4, false>", "FETCH_SIZE")]
    n, mean, median, top = table[("decode_streamk_kernel<bf16_t, 128, 4, false>", "FETCH_SIZE")]
    assert (n, median, top) == (4, 1002, 1004)
    assert mean == pytest.approx((10 + 1000 + 1002 + 1004) / 4)


def test_traffic_scales_by_the_copy_calibration(tmp_path):
    dec = "void (anonymous namespace)::decode_streamk_kernel<bf16_t, 128, 4, false>(AttnArgs)"
    mrg = "void (anonymous namespace)::merge_streamk_kernel<bf16_t, 128, 4>(AttnArgs)"
    copy = "void at::native::elementwise_kernel<128, 4>(int)"
    gib_kib = 1 << 20
    # the copy of 1 GiB counts half its bytes on FETCH_SIZE and all on WRITE_SIZE
    _counters(tmp_path / "cf", [(copy, "FETCH_SIZE", gib_kib / 2)] * 3)
    _counters(tmp_path / "cw", [(copy, "WRITE_SIZE", gib_kib)] * 3)
    _counters(tmp_path / "f", [(dec, "FETCH_SIZE", 100.0), (dec, "FETCH_SIZE", 100.0),
                               (mrg, "FETCH_SIZE", 3.0), (copy, "FETCH_SIZE", 9e9)])
    _counters(tmp_path / "w", [(dec, "WRITE_SIZE", 7.0), (mrg, "WRITE_SIZE", 1.0)])
    rep = profiling.traffic(*(str(tmp_path / d) for d in ("f", "w", "cf", "cw")), "streamk")
    assert rep["calibration"] == {"fetch_scale": 2.0, "write_scale": 1.0}
    assert rep["kernels"] == {"decode_streamk_kernel": (200 + 7) * 1024,
                              "merge_streamk_kernel": (6 + 1) * 1024}
    assert rep["bytes_per_launch"] == 214 * 1024
