"""Host logic of bench.py's counter-derived traffic (no GPU): per-dispatch
means of rocprofv3 FETCH_SIZE / WRITE_SIZE rows, scaled by the calibration
copy, per phase kernel; kernels a workload does not launch are left out."""
import csv
import json
import os

import bench

ERR = "void pcd::phase_kernel<float, 64, 64, 0>(pcd::ProblemSet, pcd::PhaseArgs)"
UPD = "void pcd::phase_kernel<float, 64, 64, 1>(pcd::ProblemSet, pcd::PhaseArgs)"
COPY = "void at::native::elementwise_kernel<MulFunctor<float>>(int)"


def _write(directory, rows):
    os.makedirs(directory, exist_ok=True)
    with open(os.path.join(directory, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"], r)))


def test_traffic_from_pmc(tmp_path):
    d = str(tmp_path)
    # calibration: 1 GiB copy; FETCH_SIZE reads half the bytes (split over two instance rows), WRITE_SIZE all
    _write(f"{d}/cf", [(7, COPY, "FETCH_SIZE", 262144), (7, COPY, "FETCH_SIZE", 262144)])
    _write(f"{d}/cw", [(7, COPY, "WRITE_SIZE", 1048576)])
    # two error-phase dispatches (100 and 300 KiB fetched), one update dispatch; no plain GEMM
    _write(f"{d}/f", [(1, ERR, "FETCH_SIZE", 60), (1, ERR, "FETCH_SIZE", 40), (2, ERR, "FETCH_SIZE", 300),
                      (3, UPD, "FETCH_SIZE", 10), (4, COPY, "FETCH_SIZE", 999)])
    _write(f"{d}/w", [(1, ERR, "WRITE_SIZE", 50), (2, ERR, "WRITE_SIZE", 50), (3, UPD, "WRITE_SIZE", 8)])
    out = f"{d}/traffic.json"
    bench.traffic_from_pmc("t", f"{d}/f", f"{d}/w", f"{d}/cf", f"{d}/cw", "cmd", out_path=out)
    t = json.load(open(out))
    assert abs(t["calibration"]["fetch_factor"] - 0.5) < 1e-12 and t["calibration"]["write_factor"] == 1.0
    e = t["kernels"]["error_phase"]
    assert e["dispatches"] == [2, 2]
    assert e["fetch_bytes"] == 200 * 1024 / 0.5 and e["write_bytes"] == 50 * 1024
    assert e["bytes_per_launch"] == e["fetch_bytes"] + e["write_bytes"]
    assert t["kernels"]["update_phase"]["bytes_per_launch"] == 10 * 1024 / 0.5 + 8 * 1024
    assert "plain" not in t["kernels"]
