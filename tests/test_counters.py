"""CPU tests of the rocprofv3 counter summaries (qwen_megakernel/counters.py) on small
synthetic CSVs in rocprofv3's ``-f csv`` counter-collection layout."""

import csv

import pytest

from qwen_megakernel import counters

FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
SHORT = "void qmk::decode_kernel<qmk::Qwen3_0_6B, false, false>(qmk::KArgs)"
LONG = "void qmk::decode_kernel<qmk::Qwen3_0_6B, false, true>(qmk::KArgs)"


def _write(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for i, (k, c, v) in enumerate(rows):
            w.writerow({"Dispatch_Id": i, "Kernel_Name": k, "Counter_Name": c, "Counter_Value": v})


def test_traffic_scales_by_the_calibration_copy(tmp_path):
    f, w = tmp_path / "f.csv", tmp_path / "w.csv"
    copy = "__amd_rocclr_copyBuffer"
    _write(f, [(copy, "FETCH_SIZE", 524288.0), (SHORT, "FETCH_SIZE", 10.0), (SHORT, "FETCH_SIZE", 1000.0),
               (SHORT, "FETCH_SIZE", 2000.0)])
    _write(w, [(copy, "WRITE_SIZE", 1048576.0), (SHORT, "WRITE_SIZE", 5.0), (SHORT, "WRITE_SIZE", 3.0),
               (SHORT, "WRITE_SIZE", 5.0)])
    t = counters.traffic(str(f), str(w), timed=2)
    assert t["fetch"]["scale"] == 2.0 and t["fetch"]["bytes"] == 1500 * 1024 * 2
    assert t["write"]["bytes"] == 4 * 1024
    assert t["total_bytes"] == 1500 * 1024 * 2 + 4 * 1024


def test_traffic_needs_the_calibration_copy(tmp_path):
    f = tmp_path / "f.csv"
    _write(f, [(SHORT, "FETCH_SIZE", 10.0)])
    with pytest.raises(ValueError, match="calibration"):
        counters.traffic(str(f), str(f), timed=1)


def test_sq_summary_per_instantiation_and_ratios(tmp_path):
    a, b = tmp_path / "a.csv", tmp_path / "b.csv"
    rows = []
    for i in range(3):  # the first dispatch of each kernel is outside the timed window
        rows += [(SHORT, "SQ_LDS_BANK_CONFLICT", 100.0 * (i + 1)), (SHORT, "SQ_ACTIVE_INST_LDS", 1000.0),
                 (SHORT, "GRBM_GUI_ACTIVE", 50.0), (LONG, "SQ_LDS_BANK_CONFLICT", 0.0),
                 (LONG, "SQ_ACTIVE_INST_LDS", 10.0)]
    _write(a, rows)
    _write(b, [(SHORT, "SQ_WAIT_ANY", 30.0), (SHORT, "SQ_WAVE_CYCLES", 40.0)] * 3 + [("other_kernel", "SQ_WAIT_ANY", 1.0)])
    s = counters.sq_summary([str(a), str(b)], timed=2)
    assert set(s) == {"decode_kernel<qmk::Qwen3_0_6B, false, false>", "decode_kernel<qmk::Qwen3_0_6B, false, true>"}
    short = s["decode_kernel<qmk::Qwen3_0_6B, false, false>"]
    assert short["dispatches"] == 3
    assert short["mean"]["SQ_LDS_BANK_CONFLICT"] == 250.0  # mean of the last two
    assert short["lds_bank_conflict_per_active_cycle"] == 0.25
    assert short["LDSBankConflict_pct"] == round(100 * 250.0 / (50.0 / 8) / 256, 4)  # GRBM summed over 8 XCDs
    assert short["wait_share"] == 0.75
    assert s["decode_kernel<qmk::Qwen3_0_6B, false, true>"]["lds_bank_conflict_per_active_cycle"] == 0.0
