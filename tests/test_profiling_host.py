"""The rocprofv3 CSV readers and the tile-timeline report of aster_amd.profiling, on
hand-made counter files and trace marks."""

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


def test_tile_timeline_report_from_marks():
    np = pytest.importorskip("numpy")
    # two tile units of four waves (marks in 100 MHz ticks, info: steps, XCC, kv head,
    # range); unused trace slots stay zero and are dropped
    marks = np.zeros((12, 8), np.int64)
    info = np.zeros((12, 4), np.int32)
    for w in range(8):
        t0 = 1000 + 10 * w  # wave w starts 0.1 w us after the first
        # checked +2 us, queries +1 us, first step +3 us, 7 later steps of 2 us, store 1 us
        marks[w, :6] = [t0, t0 + 200, t0 + 300, t0 + 600, t0 + 2000, t0 + 2100]
        info[w] = [8, w // 4, w // 4, 0]
    rep = profiling._tiles_report(marks, info, decode_start=1000 + 70 + 2100 + 350)
    assert rep["waves"] == 8 and rep["steps_per_unit"] == [8.0, 8.0, 8.0]
    assert rep["start_us"] == [0.0, 0.35, 0.7]
    assert rep["checked_us"] == [2.0, 2.0] and rep["queries_us"] == [1.0, 1.0]
    assert rep["first_step_us"] == [3.0, 3.0] and rep["later_step_us"] == 2.0
    assert rep["store_us"] == [1.0, 1.0]
    assert rep["exit_pct_50_90_100_us"][2] == 21.7
    assert rep["per_xcc_max_exit"] == {0: 21.3, 1: 21.7}
    assert rep["decode_first_wave_after_last_tile_us"] == 3.5
