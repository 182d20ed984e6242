"""bench_pmc.py's bookkeeping on the CPU: kernel names, counter files, the
copy calibration, traffic per launch and the --merge rule. The rocprofv3 runs
are replaced by CSV files of the shape rocprofv3 writes."""
from __future__ import annotations

import csv
import json
import os
import sys

import pytest

import bench_pmc as B


def test_kernel_base_strips_return_type_and_parameters():
    assert B.kernel_base("void moe_gu_grouped_kernel<false>(MoeDev)") == "moe_gu_grouped_kernel<false>"
    assert B.kernel_base("moe_sort_kernel(MoeDev)") == "moe_sort_kernel"
    # parentheses inside template arguments stay
    assert B.kernel_base("void k<(int)3, f(x)>(int, float)") == "k<(int)3, f(x)>"
    assert B.kernel_base("  gemv_raw_kernel<2, 1, true, 16, false>(unsigned char const*, int) ") == \
        "gemv_raw_kernel<2, 1, true, 16, false>"


def _counter_csv(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for d, k, c, v in rows:
            w.writerow({"Dispatch_Id": d, "Kernel_Name": k, "Counter_Name": c, "Counter_Value": v})


def _stats_csv(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Name", "Calls", "AverageNs"])
        w.writeheader()
        for n, c, a in rows:
            w.writerow({"Name": n, "Calls": c, "AverageNs": a})


def test_read_counters_means_and_last_three_copies(tmp_path):
    rows = [(1, "void kern(MoeDev)", "FETCH_SIZE", 100.0), (2, "void kern(MoeDev)", "FETCH_SIZE", 300.0)]
    # five copies: only the last three (by dispatch id) calibrate
    rows += [(10 + i, "__amd_rocclr_copyBuffer", "FETCH_SIZE", v) for i, v in enumerate([1.0, 2.0, 10.0, 20.0, 30.0])]
    _counter_csv(tmp_path / "p_counter_collection.csv", rows)
    res, calib = B.read_counters(str(tmp_path))
    assert res["kern"]["FETCH_SIZE"] == (200.0, 2)
    assert calib["FETCH_SIZE"] == pytest.approx(20.0)


def test_read_stats(tmp_path):
    _stats_csv(tmp_path / "p_kernel_stats.csv", [("void kern(MoeDev)", 7, 1500.0)])
    assert B.read_stats(str(tmp_path)) == {"kern": (1500.0, 7)}


def _fake_run_pass(fetch_kib, write_kib, copy_fetch_kib):
    """A stand-in for run_pass: writes the CSV files one rocprofv3 pass would leave."""
    def run_pass(workload, pas, raw, timeout):
        out = os.path.join(raw, f"{workload}_{pas}")
        os.makedirs(out, exist_ok=True)
        if pas == "trace":
            _stats_csv(os.path.join(out, "p_kernel_stats.csv"), [("void kern(MoeDev)", 4, 2000.0)])
            return out
        rows = []
        if pas == "fetch":
            rows = [(1, "void kern(MoeDev)", "FETCH_SIZE", fetch_kib)]
            rows += [(10 + i, "__amd_rocclr_copyBuffer", "FETCH_SIZE", copy_fetch_kib) for i in range(3)]
        elif pas == "write":
            rows = [(1, "void kern(MoeDev)", "WRITE_SIZE", write_kib)]
            rows += [(10 + i, "__amd_rocclr_copyBuffer", "WRITE_SIZE", B.COPY_KIB) for i in range(3)]
        else:
            rows = [(1, "void kern(MoeDev)", "SQ_INSTS_VALU", 5.0)]
        _counter_csv(os.path.join(out, "p_counter_collection.csv"), rows)
        return out
    return run_pass


def _main(monkeypatch, tmp_path, workloads, digest, merge, fetch_kib=1024.0):
    import bench
    monkeypatch.setattr(bench, "csrc_digest", lambda: digest)
    monkeypatch.setattr(B, "run_pass", _fake_run_pass(fetch_kib, 512.0, B.COPY_KIB / 2))
    args = ["bench_pmc.py", "--workloads", workloads, "--raw", str(tmp_path / "raw"),
            "--json", str(tmp_path / "pmc.json"), "--md", str(tmp_path / "pmc.md")]
    monkeypatch.setattr(sys, "argv", args + (["--merge"] if merge else []))
    B.main()
    with open(tmp_path / "pmc.json") as f:
        return json.load(f)


def test_traffic_from_calibrated_counters(monkeypatch, tmp_path):
    doc = _main(monkeypatch, tmp_path, "w1", "d0", merge=False)
    rec = doc["workloads"]["w1"]
    # the copy reads half its bytes through FETCH_SIZE: factor 2; WRITE_SIZE all of them: factor 1
    assert rec["fetch_factor"] == pytest.approx(2.0) and rec["write_factor"] == pytest.approx(1.0)
    k = rec["kernels"]["kern"]
    assert k["traffic_bytes"] == int(1024.0 * 1024 * 2 + 512.0 * 1024)
    assert k["avg_us"] == 2.0 and k["calls"] == 4 and k["SQ_INSTS_VALU"] == 5.0
    assert doc["csrc_digest"] == "d0"
    assert "kern" in (tmp_path / "pmc.md").read_text()


def test_merge_keeps_workloads_of_the_same_sources_only(monkeypatch, tmp_path):
    _main(monkeypatch, tmp_path, "w1", "d0", merge=False)
    doc = _main(monkeypatch, tmp_path, "w2", "d0", merge=True)
    assert set(doc["workloads"]) == {"w1", "w2"}
    # other sources: the earlier workloads are dropped, not mixed in
    doc = _main(monkeypatch, tmp_path, "w3", "d1", merge=True)
    assert set(doc["workloads"]) == {"w3"}
    # without --merge a run starts afresh
    doc = _main(monkeypatch, tmp_path, "w4", "d1", merge=False)
    assert set(doc["workloads"]) == {"w4"}
