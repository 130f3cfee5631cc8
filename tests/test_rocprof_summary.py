"""The counter-summary arithmetic behind roofline.traffic (CPU only)."""
import csv

from attentionfuse_amd import rocprof_summary as R

FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value",
          "Start_Timestamp", "End_Timestamp"]


def _write(d, rows):
    d.mkdir()
    with open(d / "run_counter_collection.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, FIELDS)
        w.writeheader()
        for i, (name, ctr, val) in enumerate(rows):
            w.writerow({"Dispatch_Id": i, "Kernel_Name": name, "Counter_Name": ctr,
                        "Counter_Value": val, "Start_Timestamp": 0, "End_Timestamp": 1000})


def test_traffic_scaled_by_copy(tmp_path):
    k = "void af::fwd_kernel<af::F16, 64, 1, 0, 0, true, 4>(af::FwdParams)"
    _write(tmp_path / "f", [(k, "FETCH_SIZE", 100.0), (k, "FETCH_SIZE", 300.0),
                            ("other", "FETCH_SIZE", 9e9)])
    _write(tmp_path / "w", [(k, "WRITE_SIZE", 50.0)])
    # the copy of 2 MiB reads as 1024 KiB fetched (factor 2) and 2048 KiB written
    _write(tmp_path / "cf", [("void at::native::neg_kernel(x)", "FETCH_SIZE", 1024.0)])
    _write(tmp_path / "cw", [("void at::native::neg_kernel(x)", "WRITE_SIZE", 2048.0)])
    out = R.traffic(str(tmp_path / "f"), str(tmp_path / "w"), str(tmp_path / "cf"),
                    str(tmp_path / "cw"), 2 << 20, ["af::"])
    assert "factor 2.0000" in out[0] and "factor 1.0000" in out[0]
    line = [x for x in out if x.startswith("TRAFFIC")]
    assert line == ["TRAFFIC af::fwd_kernel<af::F16, 64, 1, 0, 0, true, 4> "
                    f"fetch_bytes={200 * 1024 * 2} write_bytes={50 * 1024} "
                    f"total_bytes={200 * 1024 * 2 + 50 * 1024}"]


def test_mfma_fraction(tmp_path):
    k = "void af::fwd_kernel<af::F16, 64, 1, 0, 0, true, 4>(af::FwdParams)"
    # 8 XCDs x 1000 cycles; 1024 SIMDs half busy
    _write(tmp_path / "m", [(k, "GRBM_GUI_ACTIVE", 8000.0),
                            (k, "SQ_VALU_MFMA_BUSY_CYCLES", 512000.0)])
    out = "\n".join(R.pmc([str(tmp_path / "m")], ["af::"]))
    assert "MFMA busy fraction 0.500" in out and "clock 1.00 GHz" in out
