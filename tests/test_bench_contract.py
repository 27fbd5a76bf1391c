"""bench.py's host-side contract, checked without a GPU: it refuses more than one GPU with a
JSON message, and the counter summary behind ``roofline.traffic`` scales each counter by what
it reads for the calibration copy of known size."""
import csv
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], cwd=ROOT,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def _counter_csv(path, counter, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name",
                                          "Counter_Value"])
        w.writeheader()
        for i, (name, values) in enumerate(rows):
            for v in values:  # one row per XCD / instance, summed per dispatch
                w.writerow({"Dispatch_Id": i, "Kernel_Name": name, "Counter_Name": counter,
                            "Counter_Value": v})


def test_pmc_summary_copy_calibration(tmp_path):
    """GEMV-family KiB per dispatch are averaged, then divided by the factor the calibration
    copy gives (its counter reading over its known size): a counter that reads 2x the true
    bytes on the copy reads 2x on the GEMVs too."""
    sys.path.insert(0, str(ROOT))
    import bench
    calib_mib = 4
    fetch, write = tmp_path / "fetch.csv", tmp_path / "write.csv"
    # fetch counter over-reads 2x: copy of 4 MiB reads 8192 KiB; GEMVs read 300 and 500 KiB
    _counter_csv(fetch, "FETCH_SIZE", [("gemv_xreg_kernel<...>", [100.0, 200.0]),
                                       ("gemv_xlds_kernel<...>", [500.0]),
                                       ("other_kernel", [9999.0]),
                                       ("copy_bytes_kernel", [4096.0, 4096.0])])
    # write counter exact: copy reads 4096 KiB; GEMVs write 16 and 48 KiB
    _counter_csv(write, "WRITE_SIZE", [("gemv_xreg_kernel<...>", [16.0]),
                                       ("gemv_fused_kernel<...>", [48.0]),
                                       ("copy_bytes_kernel", [4096.0])])
    out = bench.pmc_summary(str(fetch), str(write), calib_mib)
    assert out["fetch"]["gemv_dispatches"] == 2 and out["write"]["gemv_dispatches"] == 2
    assert out["fetch"]["factor"] == 2.0 and out["write"]["factor"] == 1.0
    assert out["fetch"]["bytes_per_gemv_launch"] == 400 * 1024 // 2
    assert out["write"]["bytes_per_gemv_launch"] == 32 * 1024
    assert out["traffic_bytes_per_launch"] == 200 * 1024 + 32 * 1024
