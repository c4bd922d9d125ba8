"""bench.py's counter summary: the HBM traffic of the B=4096 segment kernel
from a FETCH_SIZE and a WRITE_SIZE rocprofv3 run, each counter scaled by
what it reads for the calibration copy of 1 GiB (the copy kernel's largest
dispatch), and the LM-head kernels' bytes per (kernel, grid).  Runs on
synthetic counter files written in rocprofv3's csv layout."""
import csv
import json

import numpy as np

import bench

FIELDS = ["Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"]


def _write(folder, counter, rows):
    folder.mkdir()
    with open(folder / "run_counter_collection.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=FIELDS)
        w.writeheader()
        for name, grid, value in rows:
            w.writerow({"Kernel_Name": name, "Grid_Size": grid, "Counter_Name": counter,
                        "Counter_Value": value})


def test_traffic_summary(tmp_path, monkeypatch):
    seg = "void pb::segment_kernel<8, true>(pb::RowParams)"
    gemm = "void pb::lm_gemm_kernel<false>(pb::LmParams)"
    _write(tmp_path / "F", "FETCH_SIZE", [
        ("__amd_rocclr_copyBuffer", 512, 2.5),          # a small copy of the bench
        ("__amd_rocclr_copyBuffer", 131072, 524288.0),  # the 1 GiB calibration copy
        (seg, 1048576, 1000000.0), (seg, 1048576, 1000002.0),
        (seg, 8192, 7.0),                               # B=1: another grid, ignored
        (gemm, 1215488, 40000.0),
        ("void pb::lm_pack_kernel(x)", 4254208, 9.0)])
    _write(tmp_path / "W", "WRITE_SIZE", [
        ("__amd_rocclr_copyBuffer", 512, 1.0),
        ("__amd_rocclr_copyBuffer", 131072, 1048576.0),
        (seg, 1048576, 16.0), (gemm, 1215488, 150000.0)])
    out = tmp_path / "traffic.json"
    monkeypatch.setattr(bench, "PMC_SUMMARY", out)
    from promptboot_amd import sampler as s
    from promptboot_amd import workloads

    class FakeLib:
        @staticmethod
        def pb_version():
            return b"pbsample test"

    monkeypatch.setattr(s, "lib", lambda: FakeLib())
    monkeypatch.setattr(workloads, "make", lambda name: {"hist_len": np.full(4096, 1000, np.uint32)})
    bench.traffic_summary(str(tmp_path / "F"), str(tmp_path / "W"))
    d = json.loads(out.read_text())
    assert d["library"] == "pbsample test"
    assert d["calibration"]["fetch_scale"] == 2.0 and d["calibration"]["write_scale"] == 1.0
    assert d["segment_kernel_per_dispatch"]["dispatches"] == [2, 1]
    assert d["hbm_bytes_per_launch"] == round((1000001.0 * 2 + 16.0) * 1024)
    alg = workloads.algorithmic_bytes(np.full(4096, 1000, np.uint32))
    assert d["algorithmic_bytes_per_launch"] == alg
    (lm,) = d["lm_head_kernels_per_dispatch"]
    assert lm["kernel"] == "pb::lm_gemm_kernel<false>" and lm["grid_threads"] == 1215488
    assert (lm["fetch_bytes"], lm["write_bytes"]) == (80000 * 1024, 150000 * 1024)
    # the measured-traffic lookup takes the summary only for the same build
    assert bench.measured_traffic("pbsample test")["traffic"] == d["hbm_bytes_per_launch"]
    assert bench.measured_traffic("pbsample other")["traffic"] is None
