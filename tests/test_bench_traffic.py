"""bench.py's traffic derivation from rocprofv3 counter files (CPU only).

The four counter runs are written here as small CSV files in rocprofv3's
counter_collection layout; the derived bytes follow from the copy's scale.
"""
from __future__ import annotations

import csv
import json

import bench

FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def write_run(path, counter, rows):
    path.mkdir()
    with open(path / "run_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for i, (kernel, value) in enumerate(rows):
            w.writerow({"Dispatch_Id": i, "Kernel_Name": kernel, "Counter_Name": counter, "Counter_Value": value})


def test_traffic_scales_each_counter_by_the_copy(tmp_path):
    gib_kib = (1 << 30) / 1024
    # the copy reads 1 GiB and writes 1 GiB; FETCH_SIZE counts half of its reads here
    write_run(tmp_path / "pmc_copy_FETCH_SIZE", "FETCH_SIZE",
              [("__amd_rocclr_fillBufferAligned", 40.0), ("(anonymous namespace)::hbm_copy_kernel(...)", gib_kib / 2)] * 2)
    write_run(tmp_path / "pmc_copy_WRITE_SIZE", "WRITE_SIZE",
              [("(anonymous namespace)::hbm_copy_kernel(...)", gib_kib)])
    write_run(tmp_path / "pmc_step_FETCH_SIZE", "FETCH_SIZE",
              [("leafhip::decode_step_kernel(StepParams)", 1000.0), ("leafhip::decode_step_kernel(StepParams)", 3000.0),
               ("leafhip::norm_kernel(...)", 5.0e6)])
    write_run(tmp_path / "pmc_step_WRITE_SIZE", "WRITE_SIZE",
              [("leafhip::decode_step_kernel(StepParams)", 10.0)])
    out = bench.derive_traffic(tmp_path)
    # mean 2000 KiB counted x 2048 bytes per counted KiB, plus 10 KiB x 1024
    assert out["FETCH_SIZE"]["bytes"] == 2000 * 2048
    assert out["WRITE_SIZE"]["bytes"] == 10 * 1024
    assert out["bytes_per_launch"] == 2000 * 2048 + 10 * 1024
    json.dumps(out)


def test_committed_traffic_file_matches_its_parts():
    if not bench.TRAFFIC_FILE.exists():
        return
    t = json.loads(bench.TRAFFIC_FILE.read_text())
    assert t["kernel"] == "decode_step_kernel"
    assert abs(t["FETCH_SIZE"]["bytes"] + t["WRITE_SIZE"]["bytes"] - t["bytes_per_launch"]) <= 1
