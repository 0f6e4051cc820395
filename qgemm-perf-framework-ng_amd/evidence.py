#!/usr/bin/env python3
"""rocprofv3 evidence for the MI355X backend: one configuration, one counter
set, a Markdown/JSON report with roofline fractions.

Two sub-commands, so that the profiler itself is started from the command line
(the program goes right after `rocprofv3 ... --`):

  workload   runs one baseline configuration with plain launches on the
             current stream, then one device copy of 256 MiB (the calibration
             kernel: it must fetch and write exactly that many bytes).
  summarize  reads the CSV output of one --kernel-trace --stats run and of
             two --pmc runs (FETCH_SIZE, then WRITE_SIZE), and reports for the
             configuration's kernel: average duration, algorithmic bytes and
             ops, HBM bytes per launch (counter KiB x the copy calibration
             factor), and the fractions of the 8 TB/s and 5.0 POPS peaks.
             Optional --sq runs (SQ_ counters, at most 8 per run) add the
             per-dispatch counters and, for the GEMMs, the VALU / MFMA / LDS
             wave-instructions per item (one 32x32x32 int8 MFMA tile, 65536
             ops): the VALU work an item needs against the 32 cycles of its
             int8 MFMA, and the cycles per item the run achieved per SIMD.

Example (the three profiler passes, then the summary):
  python3 qgemm-perf-framework-ng_amd/evidence.py workload --config c1 --iters 200   # under rocprofv3
  python3 qgemm-perf-framework-ng_amd/evidence.py summarize --config c1 \\
      --trace OUT/trace --fetch OUT/fetch --write OUT/write --md profiles/x.md --json profiles/traffic.json
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
COPY_BYTES = 256 << 20
SIMDS = 256 * 4            # MI355X: 256 CUs of 4 SIMDs
PEAK_CLOCK_GHZ = 2.4       # the clock the published peaks assume
ITEM_OPS = 2 * 32 * 32 * 32
VALU_CYCLES_PER_INST = 4   # a wave64 VALU instruction on a 16-lane SIMD (no packed fp32)
MFMA_CYCLES_PER_ITEM = 32  # v_mfma_i32_32x32x32_i8 at the 5.0 POPS peak

# name, qtype, m, n, k, input variant, kernel-name substring, bound
CONFIGS = {
    "c0": ("q4_0 x q8_0 GEMM M=480 N=1536 K=1536", 0, 480, 1536, 1536, 0, "gemm_q4_0_wt_kernel", "mfma"),
    "c1": ("q4_0 x q8_0 GEMV M=1 N=4096 K=4096, 48 rotating weight copies", 0, 1, 4096, 4096, 0,
           "gemv_q4_0_m1_kernel", "hbm"),
    "c2": ("q4_K x q8_K GEMM M=480 N=1536 K=1536", 1, 480, 1536, 1536, 0, "gemm_q4_K_wt_kernel", "mfma"),
    "c3": ("iq2_xxs x q8_K GEMM M=512 N=4096 K=4096 (baseline weight generator)", 2, 512, 4096, 4096, 1,
           "gemm_kq_kernel", "mfma"),
    "c4": ("q4_0 x q8_0 GEMM M=2048 N=11008 K=4096", 0, 2048, 11008, 4096, 0, "gemm_q4_0_kernel", "mfma"),
    # decode batches (not baseline configurations): at K = 4096 M = 8 and 16 run the MFMA tile GEMVs
    # (one chunk of the chunked kernels; iq2_xxs at M = 8 the two-half-copy kernel)
    "m8_q4_0": ("q4_0 x q8_0 GEMV M=8 N=4096 K=4096, 48 rotating weight copies", 0, 8, 4096, 4096, 0,
                "gemv_q4_0_mfma_chunk_kernel", "hbm"),
    "m8_q4_K": ("q4_K x q8_K GEMV M=8 N=4096 K=4096, 48 rotating weight copies", 1, 8, 4096, 4096, 0,
                "gemv_q4_K_mfma_chunk_kernel", "hbm"),
    "m8_iq2_xxs": ("iq2_xxs x q8_K GEMV M=8 N=4096 K=4096, 48 rotating weight copies", 2, 8, 4096, 4096, 1,
                   "gemv_iq2_xxs_mfma_sb_kernel", "hbm"),
    "m16_q4_0": ("q4_0 x q8_0 GEMV M=16 N=4096 K=4096, 48 rotating weight copies", 0, 16, 4096, 4096, 0,
                 "gemv_q4_0_mfma_chunk_kernel", "hbm"),
    "m16_q4_K": ("q4_K x q8_K GEMV M=16 N=4096 K=4096, 48 rotating weight copies", 1, 16, 4096, 4096, 0,
                 "gemv_q4_K_mfma_chunk_kernel", "hbm"),
    "m16_iq2_xxs": ("iq2_xxs x q8_K GEMV M=16 N=4096 K=4096, 48 rotating weight copies", 2, 16, 4096, 4096, 1,
                    "gemv_iq2_xxs_mfma_chunk_kernel", "hbm"),
    # the M = 1 GEMVs of the other two formats (bench.py's gemv_q4_K / gemv_iq2_xxs lines)
    "m1_q4_K": ("q4_K x q8_K GEMV M=1 N=4096 K=4096, 48 rotating weight copies", 1, 1, 4096, 4096, 0,
                "gemv_q4_K_kernel", "hbm"),
    "m1_iq2_xxs": ("iq2_xxs x q8_K GEMV M=1 N=4096 K=4096, 48 rotating weight copies", 2, 1, 4096, 4096, 1,
                   "gemv_iq2_xxs_kernel", "hbm"),
}
WB = {0: 18, 1: 144, 2: 66}
AB = {0: 34, 1: 292, 2: 292}
QK = {0: 32, 1: 256, 2: 256}


def algorithmic(cfg):
    _, qt, m, n, k, _, _, _ = CONFIGS[cfg]
    nb = k // QK[qt]
    return {"bytes": n * nb * WB[qt] + m * nb * AB[qt] + m * n * 4, "ops": 2.0 * m * n * k}


def load_package():
    import importlib.util
    name = "qgemm_perf_framework_ng_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(HERE, "__init__.py"),
                                                  submodule_search_locations=[HERE])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def run_workload(cfg, iters):
    import torch
    pkg = load_package()
    label, qt, m, n, k, variant, _, _ = CONFIGS[cfg]
    print(f"[evidence] {cfg}: {label}, {iters} launches", flush=True)
    act, w = pkg.create_input(qt, m, n, k, seed=1, variant=variant)
    copies = 48 if CONFIGS[cfg][7] == "hbm" else 1  # GEMVs: more weight bytes (453 MB) than the 256 MB MALL holds
    base = torch.from_numpy(w).cuda()
    weights = [base] + [base.clone() for _ in range(copies - 1)]
    aq = pkg.quantize_activation(qt, torch.from_numpy(act).cuda())
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    for i in range(iters):
        pkg.mul_mat(qt, weights[i % copies], aq, m, n, k, out=out)
    torch.cuda.synchronize()
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[evidence] done ({COPY_BYTES >> 20} MiB calibration copy)", flush=True)


def read_csvs(root, suffix):
    rows = []
    for path in sorted(glob.glob(os.path.join(root, "**", f"*{suffix}"), recursive=True)):
        with open(path, newline="") as f:
            rows.extend(csv.DictReader(f))
    return rows


def counter_per_dispatch(rows, counter, match):
    vals = [float(r["Counter_Value"]) for r in rows if r.get("Counter_Name") == counter and match(r["Kernel_Name"])]
    return (sum(vals) / len(vals), len(vals)) if vals else (None, 0)


def calibration_copy(rows, counter):
    """Counter value of the workload's final dispatch, the 256 MiB device copy
    (earlier copy kernels are the uploads and weight clones)."""
    mine = [r for r in rows if r.get("Counter_Name") == counter]
    if not mine:
        return None
    last = max(mine, key=lambda r: int(r["Dispatch_Id"]))
    return float(last["Counter_Value"]) if "copy" in last["Kernel_Name"].lower() else None


def summarize(args):
    label, qt, m, n, k, _, kname, bound = CONFIGS[args.config]
    alg = algorithmic(args.config)
    stats = read_csvs(args.trace, "kernel_stats.csv")
    kstat = [r for r in stats if kname in r["Name"]]
    if not kstat:
        raise SystemExit(f"no kernel matching {kname} in {args.trace}")
    calls = sum(int(r["Calls"]) for r in kstat)
    avg_ns = sum(float(r["TotalDurationNs"]) for r in kstat) / calls
    kernel_full = max(kstat, key=lambda r: int(r["Calls"]))["Name"]
    report = {"config": args.config, "workload": label, "kernel": kname, "kernel_symbol": kernel_full[:160],
              "calls": calls, "avg_us": round(avg_ns / 1e3, 4)}
    # per-dispatch durations: the median and the fastest dispatch beside the
    # average (a few slow dispatches, the first ones, lift the average)
    durs = sorted((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
                  for r in read_csvs(args.trace, "kernel_trace.csv") if kname in r["Kernel_Name"])
    if durs:
        report["median_us"] = round(durs[len(durs) // 2], 4)
        report["min_us"] = round(durs[0], 4)
    report.update({"algorithmic_bytes": alg["bytes"], "algorithmic_ops": alg["ops"]})
    if bound == "hbm":
        a = alg["bytes"] / (avg_ns * 1e-9) / 1e9
        report.update({"bound": "hbm", "achieved_gbs": round(a, 2), "frac": round(a / HBM_PEAK_GBS, 4)})
    else:
        a = alg["ops"] / (avg_ns * 1e-9) / 1e12
        report.update({"bound": "mfma", "achieved_tops": round(a, 2), "frac": round(a / INT8_PEAK_TOPS, 4)})
    hbm = None
    if args.fetch and args.write:
        fr, wr = read_csvs(args.fetch, "counter_collection.csv"), read_csvs(args.write, "counter_collection.csv")
        f_k, nf = counter_per_dispatch(fr, "FETCH_SIZE", lambda s: kname in s)
        w_k, nw = counter_per_dispatch(wr, "WRITE_SIZE", lambda s: kname in s)
        f_c = calibration_copy(fr, "FETCH_SIZE")
        w_c = calibration_copy(wr, "WRITE_SIZE")
        if None not in (f_k, w_k, f_c, w_c) and f_c > 0 and w_c > 0:
            ff, fw = COPY_BYTES / (f_c * 1024), COPY_BYTES / (w_c * 1024)
            hbm = f_k * 1024 * ff + w_k * 1024 * fw
            report.update({"fetch_kib_per_dispatch": round(f_k, 1), "write_kib_per_dispatch": round(w_k, 1),
                           "dispatches_counted": [nf, nw], "copy_fetch_kib": round(f_c, 1),
                           "copy_write_kib": round(w_c, 1), "calibration_fetch": round(ff, 4),
                           "calibration_write": round(fw, 4), "hbm_bytes_per_launch": int(round(hbm)),
                           "hbm_over_algorithmic": round(hbm / alg["bytes"], 3)})
    if args.sq:
        sq = {}
        for root in args.sq:
            for r in read_csvs(root, "counter_collection.csv"):
                if kname in r["Kernel_Name"] and r.get("Counter_Name", "").startswith(("SQ_", "GRBM_")):
                    sq.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
        for name in sorted(sq):
            report[f"{name}_per_dispatch"] = round(sum(sq[name]) / len(sq[name]), 1)
        if bound == "mfma" and "SQ_INSTS_VALU" in sq:
            items = alg["ops"] / ITEM_OPS
            per = {name: sum(v) / len(v) / items for name, v in sq.items()}
            report["items_per_launch"] = int(items)
            report["valu_insts_per_item"] = round(per["SQ_INSTS_VALU"], 2)
            if "SQ_INSTS_MFMA" in per:
                report["mfma_insts_per_item"] = round(per["SQ_INSTS_MFMA"], 2)
                valu_only = per["SQ_INSTS_VALU"] - per["SQ_INSTS_MFMA"]
                report["non_mfma_valu_insts_per_item"] = round(valu_only, 2)
                report["valu_cycles_per_item"] = round(valu_only * VALU_CYCLES_PER_INST, 1)
            if "SQ_INSTS_LDS" in per:
                report["lds_insts_per_item"] = round(per["SQ_INSTS_LDS"], 2)
            report["mfma_cycles_per_item_at_peak"] = MFMA_CYCLES_PER_ITEM
            report["achieved_cycles_per_item_per_simd"] = round(
                avg_ns * 1e-9 * PEAK_CLOCK_GHZ * 1e9 * SIMDS / items, 1)
    lines = [f"# {kname} — {args.config}: {label}", "",
             "Produced by `qgemm-perf-framework-ng_amd/evidence.py summarize` from rocprofv3 runs of",
             f"`evidence.py workload --config {args.config}`.", "", "Commands:", "```"]
    lines += [c for c in (args.command or [])]
    lines += ["```", "", "| quantity | value |", "|---|---|"]
    for key, val in report.items():
        lines.append(f"| {key} | {val} |")
    if args.md:
        os.makedirs(os.path.dirname(os.path.abspath(args.md)), exist_ok=True)
        with open(args.md, "w") as f:
            f.write("\n".join(lines) + "\n")
    if args.json:
        table = {"entries": []}
        if os.path.exists(args.json):
            with open(args.json) as f:
                table = json.load(f)
        entry = {"kernel": kname if args.config != "c1" else "gemv_q4_0_m1_kernel", "workload": args.config,
                 "hbm_bytes_per_launch": report.get("hbm_bytes_per_launch"), "report": report}
        table["entries"] = [e for e in table["entries"] if e.get("workload") != args.config] + [entry]
        with open(args.json, "w") as f:
            json.dump(table, f, indent=1)
    print(json.dumps(report))


def bench_stats(args):
    """Per-kernel table of a `rocprofv3 --kernel-trace --stats -- python3 bench.py`
    run, with the bench line's own HIP-event kernel times beside the kernels
    they name (the average of every matching dispatch)."""
    stats = read_csvs(args.trace, "kernel_stats.csv")
    if not stats:
        raise SystemExit(f"no kernel_stats.csv under {args.trace}")
    line = {}
    if args.bench_json:
        with open(args.bench_json) as f:
            text = [t for t in f.read().splitlines() if t.startswith("{")]
        line = json.loads(text[-1]) if text else {}
    items = [("c1 headline", line.get("roofline"))]
    for key in ("gemm", "q4_K", "iq2_xxs", "prefill", "gemv_q4_K", "gemv_iq2_xxs"):
        if isinstance(line.get(key), dict):
            items.append((key, line[key].get("roofline")))
    for it in line.get("decode") or []:
        items.append((it["workload"].split(":")[0], it.get("roofline")))

    def short(name):
        name = name.replace("(anonymous namespace)::", "").replace("pfng::", "")
        name = name[5:] if name.startswith("void ") else name
        return name.split("(int")[0].split("(unsigned")[0].split("(float")[0].split("(__")[0][:110]

    # per-dispatch durations, for medians: under --kernel-trace a dispatch of a
    # few microseconds carries the tracer's own overhead (an empty kernel
    # records about 4.3 us), so the median is the steadier figure for them
    durations = {}
    for r in read_csvs(args.trace, "kernel_trace.csv"):
        durations.setdefault(r["Kernel_Name"], []).append(
            (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)

    def median_us(name):
        d = sorted(durations.get(name, []))
        return f"{d[len(d) // 2]:.3f}" if d else "-"

    rows = sorted(stats, key=lambda r: -float(r["TotalDurationNs"]))
    out = ["# bench.py kernel statistics (rocprofv3 --kernel-trace --stats)", "",
           "Command (repository root on the GPU box), then the summary:", "```"]
    out += list(args.command or [])
    out += ["```", "", "| kernel | calls | avg us | median us | min us | max us |", "|---|---|---|---|---|---|"]
    for r in rows:
        out.append(f"| `{short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.3f} | "
                   f"{median_us(r['Name'])} | {float(r['MinNs']) / 1e3:.3f} | {float(r['MaxNs']) / 1e3:.3f} |")
    out += ["", "Bench items (HIP events over back-to-back graph replays, unprofiled run) against the",
            "profiler's average and median for the kernel family each item names. Traced dispatches",
            "are spaced apart and carry the tracer's overhead (an empty kernel records about 4.3 us,",
            "profiles/launch_and_read_floor.md), so for kernels of a few microseconds the traced",
            "figures sit above the back-to-back ones:", "",
            "| item | kernel | bench kernel_us | profiler avg / median us (matching dispatches) |",
            "|---|---|---|---|"]
    for label, roof in items:
        if not roof:
            continue
        kname = roof["kernel"]
        base, _, tag = kname.partition("<")
        tag = tag.rstrip(">")
        # K-quant tiles are tagged by type; GEMV instantiations by their row count
        # (the first template argument, more may follow)
        tags = {"q4_K": ["(Kq)0"], "iq2_xxs": ["(Kq)1"]}.get(tag, [f"<{tag}>", f"<{tag},"] if tag.isdigit() else [""])
        match = [r for r in stats if base in r["Name"] and any(t in short(r["Name"]) for t in tags)]
        # one line per instantiation: the plan picks the tile configuration by shape
        for r in match or [None]:
            prof = (f"{float(r['AverageNs']) / 1e3:.3f} / {median_us(r['Name'])} "
                    f"(`{short(r['Name'])}`, {r['Calls']} dispatches)" if r else "not profiled")
            out.append(f"| {label} | `{kname}` | {roof['kernel_us']} | {prof} |")
    out.append("")
    with open(args.md, "w") as f:
        f.write("\n".join(out) + "\n")
    print("\n".join(out))


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="cmd", required=True)
    b = sub.add_parser("bench-stats")
    b.add_argument("--trace", required=True, help="output directory of the profiled bench.py run")
    b.add_argument("--bench-json", help="file holding the bench.py JSON line of that run")
    b.add_argument("--md", required=True)
    b.add_argument("--command", action="append", help="profiler command line to record in the summary")
    w = sub.add_parser("workload")
    w.add_argument("--config", choices=sorted(CONFIGS), required=True)
    w.add_argument("--iters", type=int, default=100)
    s = sub.add_parser("summarize")
    s.add_argument("--config", choices=sorted(CONFIGS), required=True)
    s.add_argument("--trace", required=True, help="output directory of the --kernel-trace --stats run")
    s.add_argument("--fetch", help="output directory of the --pmc FETCH_SIZE run")
    s.add_argument("--write", help="output directory of the --pmc WRITE_SIZE run")
    s.add_argument("--sq", action="append", help="output directory of an --pmc run of SQ_ counters (repeatable)")
    s.add_argument("--md", help="Markdown summary to write")
    s.add_argument("--json", help="traffic table to update")
    s.add_argument("--command", action="append", help="profiler command line to record in the summary")
    args = ap.parse_args()
    if args.cmd == "workload":
        run_workload(args.config, args.iters)
    elif args.cmd == "bench-stats":
        bench_stats(args)
    else:
        summarize(args)


if __name__ == "__main__":
    main()
