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
    """Backbone layer-tail KiB per dispatch (demangled or mangled names; the decoder's tail, the
    head launch, the last layer's tail and other kernels excluded) are averaged, then divided by the factor the calibration copy gives
    (its counter reading over its known size): a counter that reads 2x the true bytes on the
    copy reads 2x on the tail too."""
    sys.path.insert(0, str(ROOT))
    import bench
    calib_mib = 4
    fetch, write = tmp_path / "fetch.csv", tmp_path / "write.csv"
    bb = "void ecd::tail::layer_tail_kernel<6, 16, 4, 1, 128, 3, true, false, 8>(ecd::tail::Args)"
    bb_mangled = "_ZN3ecd4tail17layer_tail_kernelILi6ELi16ELi4ELi1ELi128ELi3ELb1ELb0ELi8EEEvNS0_4ArgsE"
    dec = "void ecd::tail::layer_tail_kernel<2, 16, 4, 4, 128, 4, false, false, 16>(ecd::tail::Args)"
    head = "void ecd::tail::layer_tail_kernel<6, 16, 4, 1, 128, 3, true, true, 8>(ecd::tail::Args)"
    head_mangled = "_ZN3ecd4tail17layer_tail_kernelILi6ELi16ELi4ELi1ELi128ELi3ELb1ELb1ELi8EEEvNS0_4ArgsE"
    last = "void ecd::tail::layer_tail_kernel<6, 16, 4, 1, 0, 0, true, false, 8>(ecd::tail::Args)"
    # fetch counter over-reads 2x: copy of 4 MiB reads 8192 KiB; the tails read 300, 500 and
    # 400 KiB (the decoder's tail and the backbone's head launch are not counted)
    _counter_csv(fetch, "FETCH_SIZE", [(bb, [100.0, 200.0]), (bb_mangled, [500.0]),
                                       (dec, [7777.0]), (head, [55.0]), (head_mangled, [66.0]),
                                       (last, [400.0]), ("other_kernel", [9999.0]),
                                       ("copy_bytes_kernel", [4096.0, 4096.0])])
    # write counter exact: copy reads 4096 KiB; the tails write 16 and 48 KiB
    _counter_csv(write, "WRITE_SIZE", [(bb, [16.0]), (bb_mangled, [48.0]), (last, [32.0]),
                                       (dec, [1.0]), (head, [5.0]),
                                       ("copy_bytes_kernel", [4096.0])])
    out = bench.pmc_summary(str(fetch), str(write), calib_mib)
    assert out["fetch"]["tail_dispatches"] == 3 and out["write"]["tail_dispatches"] == 3
    assert out["fetch"]["factor"] == 2.0 and out["write"]["factor"] == 1.0
    assert out["fetch"]["bytes_per_tail_launch"] == 400 * 1024 // 2
    assert out["write"]["bytes_per_tail_launch"] == 32 * 1024
    assert out["traffic_bytes_per_launch"] == 200 * 1024 + 32 * 1024


def test_pmc_gemm_summary_groups_variants(tmp_path):
    """The prompt-GEMM counter summary groups dispatches by kernel and grid, averages each
    counter over them and forms VALU per MFMA and the f16 FLOP (MOPS x 512)."""
    sys.path.insert(0, str(ROOT))
    import bench
    path = tmp_path / "c.csv"
    rows = [(1, "gemm_i8p_kernel<0>", 98304, "SQ_INSTS_MFMA", 100.0),
            (1, "gemm_i8p_kernel<0>", 98304, "SQ_INSTS_VALU", 300.0),
            (1, "gemm_i8p_kernel<0>", 98304, "SQ_INSTS_VALU_MFMA_MOPS_F16", 2.0),
            (1, "gemm_i8p_kernel<0>", 98304, "MfmaUtil", 30.0),
            (2, "gemm_i8p_kernel<0>", 98304, "SQ_INSTS_MFMA", 100.0),
            (2, "gemm_i8p_kernel<0>", 98304, "SQ_INSTS_VALU", 500.0),
            (2, "gemm_i8p_kernel<0>", 98304, "SQ_INSTS_VALU_MFMA_MOPS_F16", 2.0),
            (2, "gemm_i8p_kernel<0>", 98304, "MfmaUtil", 40.0),
            (3, "gemm_i8p_kernel<1>", 524288, "SQ_INSTS_MFMA", 50.0),
            (3, "gemm_i8p_kernel<1>", 524288, "SQ_INSTS_VALU", 100.0),
            (4, "decode_attn_kernel", 64, "SQ_INSTS_MFMA", 7.0)]
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Grid_Size",
                                          "Counter_Name", "Counter_Value"])
        w.writeheader()
        for d, n, g, c, v in rows:
            w.writerow({"Dispatch_Id": d, "Kernel_Name": n, "Grid_Size": g, "Counter_Name": c,
                        "Counter_Value": v})
    out = bench.pmc_gemm_summary(str(path))
    assert [(e["kernel"], e["dispatches"]) for e in out] == [("gemm_i8p_kernel<0>", 2),
                                                             ("gemm_i8p_kernel<1>", 1)]
    e = out[0]
    assert e["mfma_insts"] == 100.0 and e["valu_insts"] == 400.0 and e["valu_per_mfma"] == 4.0
    assert e["mfma_f16_flop"] == 1024.0 and e["MfmaUtil_pct"] == 35.0
    assert out[1]["valu_per_mfma"] == 2.0 and out[1]["mfma_f16_flop"] is None
