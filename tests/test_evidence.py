"""The rocprofv3 evidence tool's summary arithmetic on synthetic profiler CSVs
(no GPU): roofline fractions from the trace, HBM bytes from the copy
calibration, and the per-item instruction counts from SQ counter runs."""
import argparse
import csv
import importlib.util
import json
import os

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
TOOL = os.path.join(HERE, "..", "qgemm-perf-framework-ng_amd", "evidence.py")


def load_tool():
    spec = importlib.util.spec_from_file_location("pfng_evidence_tool", TOOL)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def write_csv(path, header, rows):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


KNAME = "void pfng::(anonymous namespace)::gemm_q4_0_kernel<Cfg, false>(unsigned char const*)"
COUNTER_HEADER = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def make_runs(tmp_path, avg_ns, counters):
    trace = tmp_path / "trace"
    write_csv(str(trace / "run_kernel_stats.csv"),
              ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"],
              [[KNAME, 4, 4 * avg_ns, avg_ns, 100, avg_ns, avg_ns, 0],
               ["__amd_rocclr_copyBuffer", 1, 1000, 1000, 0, 1000, 1000, 0]])
    dirs = []
    for i, group in enumerate(counters):
        d = tmp_path / f"sq{i}"
        rows = []
        for disp in range(4):
            for name, value in group.items():
                rows.append([disp + 1, KNAME, name, value])
        write_csv(str(d / "run_counter_collection.csv"), COUNTER_HEADER, rows)
        dirs.append(str(d))
    fetch, write = tmp_path / "fetch", tmp_path / "write"
    # kernel dispatches, then the 256 MiB calibration copy as the last dispatch
    write_csv(str(fetch / "run_counter_collection.csv"), COUNTER_HEADER,
              [[1, KNAME, "FETCH_SIZE", 1000.0], [2, KNAME, "FETCH_SIZE", 1000.0],
               [3, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 2 * 262144.0]])
    write_csv(str(write / "run_counter_collection.csv"), COUNTER_HEADER,
              [[1, KNAME, "WRITE_SIZE", 500.0], [2, KNAME, "WRITE_SIZE", 500.0],
               [3, "__amd_rocclr_copyBuffer", "WRITE_SIZE", 262144.0]])
    return str(trace), str(fetch), str(write), dirs


def test_summary_roofline_traffic_and_per_item_counts(tmp_path, capsys):
    ev = load_tool()
    _, qt, m, n, k, _, _, _ = ev.CONFIGS["c4"]
    ops = 2.0 * m * n * k
    items = ops / 65536
    avg_ns = 300_000.0
    counters = [{"SQ_INSTS_VALU": 41 * items, "SQ_INSTS_MFMA": 2 * items, "SQ_INSTS_LDS": 3 * items},
                {"SQ_WAVES": 5504.0, "SQ_BUSY_CYCLES": 12345.0}]
    trace, fetch, write, sq = make_runs(tmp_path, avg_ns, counters)
    md = tmp_path / "out.md"
    args = argparse.Namespace(config="c4", trace=trace, fetch=fetch, write=write, sq=sq, md=str(md),
                              json=str(tmp_path / "t.json"), command=["cmd one", "cmd two"])
    ev.summarize(args)
    rep = json.loads(capsys.readouterr().out.strip().splitlines()[-1])
    assert rep["calls"] == 4 and rep["avg_us"] == 300.0
    assert rep["achieved_tops"] == pytest.approx(ops / 300e-6 / 1e12, rel=1e-4)
    assert rep["frac"] == pytest.approx(rep["achieved_tops"] / 5000.0, abs=1e-4)
    # the copy of 256 MiB reads 512 MiB by FETCH_SIZE: factor 0.5 on fetch, 1 on write
    assert rep["calibration_fetch"] == pytest.approx(0.5)
    assert rep["calibration_write"] == pytest.approx(1.0)
    assert rep["hbm_bytes_per_launch"] == 1000 * 1024 // 2 + 500 * 1024
    assert rep["items_per_launch"] == int(items)
    assert rep["valu_insts_per_item"] == pytest.approx(41.0)
    assert rep["mfma_insts_per_item"] == pytest.approx(2.0)
    assert rep["non_mfma_valu_insts_per_item"] == pytest.approx(39.0)
    assert rep["valu_cycles_per_item"] == pytest.approx(156.0)
    assert rep["lds_insts_per_item"] == pytest.approx(3.0)
    assert rep["SQ_WAVES_per_dispatch"] == 5504.0
    # 300 us at 2.4 GHz on 1024 SIMDs, over the items of one launch
    assert rep["achieved_cycles_per_item_per_simd"] == pytest.approx(300e-6 * 2.4e9 * 1024 / items, abs=0.1)
    text = md.read_text()
    assert "cmd one" in text and "| valu_insts_per_item | 41.0 |" in text
    table = json.loads((tmp_path / "t.json").read_text())
    assert [e["workload"] for e in table["entries"]] == ["c4"]


def test_summary_without_counter_runs_reports_trace_only(tmp_path, capsys):
    ev = load_tool()
    trace, _, _, _ = make_runs(tmp_path, 4100.0, [])
    args = argparse.Namespace(config="c1", trace=trace, fetch=None, write=None, sq=None, md=None, json=None,
                              command=None)
    with pytest.raises(SystemExit):
        ev.summarize(args)  # c1's kernel is the GEMV: the GEMM-only trace has none
    capsys.readouterr()
