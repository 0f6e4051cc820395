#!/usr/bin/env python3
"""Benchmark of the MI355X quantized GGML GEMM path (one JSON line on stdout).

Metric: "q4_0×q8_0 GEMM TOPS @480×1536×1536; M=1 GEMV GB/s @4096×4096".
One step = one pass of the hot path over one batch of synthetic input:
  * value   : config 1 — q4_0 x q8_0 GEMV, M=1 N=4096 K=4096, GB/s of algorithmic
              bytes (weights + q8_0 activation + fp32 output) per second. The step
              rotates over 32 weight copies (302 MB > the 256 MB Infinity Cache), so
              the weights stream from HBM as in decode.
  * gemm    : config 0 — q4_0 x q8_0 GEMM, M=480 N=1536 K=1536, TOPS = 2*M*N*K/s,
              the other half of the compound metric.
  * q4_K, iq2_xxs, prefill: configs 2, 3 and 4 in the same form.
  * gemv_q4_K, gemv_iq2_xxs: the M=1 GEMV of the super-block formats at
    N=K=4096 (not baseline configs; reported beside the headline).
  * decode: the M=8 and M=16 GEMVs (decode batches) of all three formats at
    N=K=4096, 32 rotating weight copies (not baseline configs).
Inputs come from the product's own generator (pfng_host_create_input, the
reference harness's mt19937 draws and host quantizers). Activations are
quantized once before the timed region (the reference quantizes in prepare(),
kernels/*/adapter.cpp); an end-to-end GEMV figure that includes the GPU
quantizer is reported beside it. Inputs are resident in HBM when timing starts.

Timed region: W warm-up steps, then K steps bracketed by torch.cuda.synchronize().
Launches are replayed from a captured graph (up to 32 launches per replay) so
that host launch overhead does not pace the GPU. Kernel time per launch is
measured with HIP events on the launch stream over the same region.
Every measured configuration is verified with the reference harness's
criterion (benchmark.cpp:144-156) against the device naive path, which
reproduces llama_reference::compute bit for bit.

cpu_baseline: the reference's own llama_reference::compute (oracle/_ref, built
from /root/reference sources) timed on this host on a bounded sample (c1 and
c0, about 16 s in all): on up to 16 threads (the box's CPU share; output
columns split, bit-identical result) as `value`/`cores`, and on one thread as
`value_1core`. If oracle/_ref is absent the C restatement (oracle/) is timed
instead.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

METRIC = "q4_0×q8_0 GEMM TOPS @480×1536×1536; M=1 GEMV GB/s @4096×4096"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA (5.0 POPS)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def load_package():
    import importlib.util
    name = "qgemm_perf_framework_ng_amd"
    if name in sys.modules:
        return sys.modules[name]
    d = os.path.join(REPO, "qgemm-perf-framework-ng_amd")
    spec = importlib.util.spec_from_file_location(name, os.path.join(d, "__init__.py"), submodule_search_locations=[d])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def traffic_for(kernel, workload):
    """HBM bytes per launch of `kernel` on `workload` from the committed
    rocprofv3 --pmc summary (profiles/traffic.json, FETCH_SIZE + WRITE_SIZE
    scaled by a copy-kernel calibration), or None when it was not measured."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(path) as f:
            table = json.load(f)
    except (OSError, ValueError):
        return None
    for entry in table.get("entries", []):
        if kernel.startswith(entry.get("kernel", "\0")) and workload.startswith(entry.get("workload", "\0")):
            return entry.get("hbm_bytes_per_launch")
    return None


def gemv_bytes(m, n, k):
    return n * (k // 32) * 18 + m * (k // 32) * 34 + m * n * 4


def time_graph(torch, graph, launches_per_replay, steps, warmup):
    """Replays `graph` until `steps` launches ran; returns (wall_s, event_ms, steps_run)."""
    reps = max(1, -(-steps // launches_per_replay))
    wreps = max(1, -(-warmup // launches_per_replay))
    for _ in range(wreps):
        graph.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return t1 - t0, e0.elapsed_time(e1), reps * launches_per_replay


def capture(torch, fn, count):
    """Capture `count` calls fn(i) into one graph on a side stream, after an
    eager warm-up on the same stream."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(min(count, 3)):
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(count):
            fn(i)
    torch.cuda.synchronize()
    return g


def cpu_baseline(budget_s):
    """Time the reference's compute() on the host: c1 (GEMV) in GB/s, c0 (GEMM)
    in TOPS, on all usable cores (output columns split over threads, bitwise the
    same result) and on one core."""
    import numpy as np
    import oracle as O
    O.lib()
    use_ref = O.ref_available()
    # the GPU box's CPU share is 16 cores per GPU
    threads = max(1, min(16, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()))

    def runner(t):
        if use_ref:
            R = O.ref()
            if t == 1:
                return lambda a, ww, o, mm, nn, kk: R.ref_compute(0, O._ptr(a), O._ptr(ww), O._ptr(o), mm, nn, kk)
            return lambda a, ww, o, mm, nn, kk: R.ref_compute_threads(0, O._ptr(a), O._ptr(ww), O._ptr(o), mm, nn, kk, t)
        return lambda a, ww, o, mm, nn, kk: O.lib().pfo_compute(0, O._ptr(a), O._ptr(ww), O._ptr(o), mm, nn, kk, t)

    def timed(run, shape, seconds):
        m, n, k = shape
        act, w = O.create_input(0, m, n, k, seed=1, variant=0)
        out = np.zeros((m, n), np.float32)
        reps = 0
        t0 = time.perf_counter()
        while reps == 0 or time.perf_counter() - t0 < seconds:
            run(act, w, out, m, n, k)
            reps += 1
        return reps, time.perf_counter() - t0

    c1, c0 = (1, 4096, 4096), (480, 1536, 1536)
    res = {}
    for t in (threads, 1):
        run = runner(t)
        r1, s1 = timed(run, c1, budget_s * 0.25)
        r0, s0 = timed(run, c0, budget_s * 0.25)
        res[t] = (gemv_bytes(*c1) * r1 / s1 / 1e9, 2.0 * 480 * 1536 * 1536 * r0 / s0 / 1e12, r1, s1, r0, s0)
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    allc, one = res[threads], res[1]
    what = "llama_reference::compute (oracle/_ref)" if use_ref else "oracle/pfng_oracle.c compute"
    return {
        "value": round(allc[0], 3), "unit": "GB/s", "cores": threads, "kind": "reference" if use_ref else "port",
        "sample": (f"{what} on {cpu}, activation quantize included; {threads} threads (output columns split): "
                   f"c1 1x4096x4096 x{allc[2]} calls in {allc[3]:.1f}s, c0 480x1536x1536 x{allc[4]} in {allc[5]:.1f}s; "
                   f"1 thread: c1 x{one[2]} in {one[3]:.1f}s, c0 x{one[4]} in {one[5]:.1f}s"),
        "gemm_tops": round(allc[1], 5),
        "value_1core": round(one[0], 3),
        "gemm_tops_1core": round(one[1], 5),
    }


def upload_weights(torch, w_bytes):
    return torch.from_numpy(np.ascontiguousarray(w_bytes)).cuda()


def verify_against_naive(torch, pkg, qtype, w_t, aq_t, m, n, k, got, rows=None):
    """The reference harness's criterion (benchmark.cpp:144-156): an element fails
    when both |err| and |err|/|expected| exceed 1e-3. The expected output is the
    device naive path, which evaluates llama_reference::compute's dot products in
    their exact fp32 order. `rows` restricts the check to a row sample."""
    if rows is not None:
        aq_t = aq_t[rows].contiguous()
        got = got[rows]
        m = len(rows)
    ref = pkg.mul_mat(qtype, w_t, aq_t, m, n, k, path=pkg.PATH_NAIVE)
    torch.cuda.synchronize()
    err = (got.double() - ref.double()).abs()
    rel = err / ref.double().abs().clamp_min(1e-6)
    bad = ((err > 1e-3) & (rel > 1e-3)) | ~torch.isfinite(got)
    return {"passed": bool(bad.sum().item() == 0), "error_elements": int(bad.sum().item()),
            "compared_elements": int(got.numel()), "max_abs": float(err.max().item()),
            "max_rel": float(rel.max().item())}


def gemv_item(torch, pkg, label, qtype, m, n, k, steps, warmup, variant, kernel, copies=32):
    """One GEMV configuration: GB/s of algorithmic bytes over `steps` launches
    rotating over `copies` weight copies (so the weights stream from HBM)."""
    act, w = pkg.create_input(qtype, m, n, k, seed=1, variant=variant)
    base = upload_weights(torch, w)
    weights = [base] + [base.clone() for _ in range(copies - 1)]
    aq = pkg.quantize_activation(qtype, torch.from_numpy(act).cuda())
    outs = [torch.empty((m, n), dtype=torch.float32, device="cuda") for _ in range(copies)]
    torch.cuda.synchronize()
    g = capture(torch, lambda i: pkg.mul_mat(qtype, weights[i % copies], aq, m, n, k, out=outs[i % copies]), copies)
    wall, ev_ms, steps_run = time_graph(torch, g, copies, steps, warmup)
    qk, wb, ab = pkg.QK[qtype], pkg.WEIGHT_BLOCK_BYTES[qtype], pkg.ACT_BLOCK_BYTES[qtype]
    per_call = n * (k // qk) * wb + m * (k // qk) * ab + m * n * 4
    k_us = ev_ms * 1e3 / steps_run
    achieved = per_call / (k_us * 1e-6) / 1e9
    ver = verify_against_naive(torch, pkg, qtype, weights[0], aq, m, n, k, outs[0])
    item = {"workload": label, "value": round(per_call * steps_run / wall / 1e9, 2), "unit": "GB/s",
            "steps": steps_run, "ms_per_step": round(wall * 1e3 / steps_run, 6), "verify": ver,
            "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_for(kernel, label),
                         "kernel": kernel, "kernel_us": round(k_us, 4), "bytes_per_launch": per_call}}
    log(f"[bench] {label}: {steps_run} steps, kernel {k_us:.3f} us -> {achieved:.1f} GB/s, verify={ver['passed']}")
    del g, weights, outs
    torch.cuda.empty_cache()
    return item


def gemm_item(torch, pkg, label, qtype, m, n, k, steps, warmup, variant, kernel, rows_to_verify=None):
    """One GEMM configuration: TOPS over `steps` graph-replayed launches."""
    act, w = pkg.create_input(qtype, m, n, k, seed=1, variant=variant)
    w_t = upload_weights(torch, w)
    aq_t = pkg.quantize_activation(qtype, torch.from_numpy(act).cuda())
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    per_replay = min(32, max(1, steps))
    g = capture(torch, lambda i: pkg.mul_mat(qtype, w_t, aq_t, m, n, k, out=out), per_replay)
    wall, ev, steps_run = time_graph(torch, g, per_replay, steps, warmup)
    ops = 2.0 * m * n * k
    k_us = ev * 1e3 / steps_run
    rows = None
    if rows_to_verify is not None and rows_to_verify < m:
        rows = torch.from_numpy(np.sort(np.random.default_rng(4).choice(m, rows_to_verify, replace=False))).cuda()
    ver = verify_against_naive(torch, pkg, qtype, w_t, aq_t, m, n, k, out, rows)
    achieved = ops / (k_us * 1e-6) / 1e12
    item = {"workload": label, "value": round(ops * steps_run / wall / 1e12, 3), "unit": "TOPS", "steps": steps_run,
            "ms_per_step": round(wall * 1e3 / steps_run, 6), "verify": ver,
            "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                         "frac": round(achieved / INT8_PEAK_TOPS, 4), "traffic": traffic_for(kernel, label),
                         "kernel": kernel, "kernel_us": round(k_us, 3)}}
    log(f"[bench] {label}: {steps_run} steps, {item['value']} TOPS wall, kernel {k_us:.2f} us -> {achieved:.1f} TOPS, "
        f"verify={ver['passed']} (max_abs {ver['max_abs']:.3g})")
    del w_t, aq_t, out, g
    torch.cuda.empty_cache()
    return item


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=6400, help="timed GEMV steps (rounded up to a multiple of 32)")
    ap.add_argument("--warmup", type=int, default=640)
    ap.add_argument("--gemm-steps", type=int, default=2048, help="timed steps of the c0/c2 GEMMs")
    ap.add_argument("--iq2-steps", type=int, default=512, help="timed c3 GEMM steps (0 = skip)")
    ap.add_argument("--prefill-steps", type=int, default=64, help="timed c4 GEMM steps (0 = skip)")
    ap.add_argument("--cpu-seconds", type=float, default=16.0, help="bounded CPU-baseline budget (0 = skip)")
    ap.add_argument("--decode-steps", type=int, default=None,
                    help="timed steps of each M=8/M=16 decode GEMV (default steps/8, 0 = skip)")
    args = ap.parse_args()

    if args.gpus != 1:
        log(f"bench.py: --gpus {args.gpus} is not supported; this build runs the hot path on one MI355X "
            "(N-sharded multi-GPU operation is a design note only).")
        sys.exit(2)
    if int(os.environ.get("RANK", "0")) != 0:
        return

    import torch

    pkg = load_package()
    arch, cus = pkg.device_check()
    log(f"[bench] device {arch}, {cus} CUs; {pkg.version()}")

    # ---------------- config 1: GEMV M=1 N=4096 K=4096, rotating weights ----------------
    m, n, k = 1, 4096, 4096
    copies = 32
    act, w = pkg.create_input(0, m, n, k, seed=1, variant=pkg.INPUT_REFERENCE)
    base = upload_weights(torch, w)
    weights = [base] + [base.clone() for _ in range(copies - 1)]
    act_t = torch.from_numpy(act).cuda()
    aq = pkg.quantize_q8_0(act_t)
    outs = [torch.empty((m, n), dtype=torch.float32, device="cuda") for _ in range(copies)]
    ws = torch.empty(pkg.lib().pfng_hip_compute_workspace_size(0, m, k), dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    log(f"[bench] c1 gemv {m}x{n}x{k}: {copies} weight copies, {copies * w.nbytes / 1e6:.0f} MB resident")

    g = capture(torch, lambda i: pkg.mul_mat(0, weights[i % copies], aq, m, n, k, out=outs[i % copies]), copies)
    wall, ev_ms, steps = time_graph(torch, g, copies, args.steps, args.warmup)
    per_call = gemv_bytes(m, n, k)
    value = per_call * steps / wall / 1e9
    kernel_us = ev_ms * 1e3 / steps
    achieved = per_call / (kernel_us * 1e-6) / 1e9
    log(f"[bench] c1 gemv: {steps} steps, wall {wall * 1e3:.2f} ms, {value:.1f} GB/s; kernel {kernel_us:.3f} us "
        f"-> {achieved:.1f} GB/s")

    g2 = capture(torch, lambda i: pkg.compute(0, act_t, weights[i % copies], n, out=outs[i % copies], workspace=ws),
                 copies)
    wall2, ev2, steps2 = time_graph(torch, g2, copies, args.steps, args.warmup)
    e2e_gbs = (per_call + m * k * 4) * steps2 / wall2 / 1e9
    got = pkg.mul_mat(0, weights[0], aq, m, n, k)
    ver1 = verify_against_naive(torch, pkg, 0, weights[0], aq, m, n, k, got)
    del g, g2, weights, outs
    torch.cuda.empty_cache()

    # ---------------- GEMM configs ----------------
    gemm = gemm_item(torch, pkg, "c0: q4_0 x q8_0 GEMM M=480 N=1536 K=1536", 0, 480, 1536, 1536, args.gemm_steps, 256,
                     pkg.INPUT_REFERENCE, "gemm_q4_0_kernel")
    q4k = gemm_item(torch, pkg, "c2: q4_K x q8_K GEMM M=480 N=1536 K=1536", 1, 480, 1536, 1536, args.gemm_steps, 256,
                    pkg.INPUT_REFERENCE, "gemm_kq_kernel<q4_K>")
    iq2 = None
    if args.iq2_steps > 0:
        iq2 = gemm_item(torch, pkg, "c3: iq2_xxs x q8_K GEMM M=512 N=4096 K=4096 (baseline weight generator)", 2, 512,
                        4096, 4096, args.iq2_steps, 32, pkg.INPUT_BASELINE, "gemm_kq_kernel<iq2_xxs>")
    prefill = None
    if args.prefill_steps > 0:
        prefill = gemm_item(torch, pkg, "c4: q4_0 x q8_0 GEMM M=2048 N=11008 K=4096", 0, 2048, 11008, 4096,
                            args.prefill_steps, 8, pkg.INPUT_REFERENCE, "gemm_q4_0_kernel", rows_to_verify=256)

    gemv_kq = [gemv_item(torch, pkg, f"m1_{name}: {name} x q8_K GEMV M=1 N=4096 K=4096, 32 rotating weight copies", qt, 1, 4096,
                         4096, args.steps // 4, args.warmup // 4, variant, f"gemv_{name}_kernel<1>")
               for qt, name, variant in ((1, "q4_K", pkg.INPUT_REFERENCE), (2, "iq2_xxs", pkg.INPUT_BASELINE))]

    decode_steps = args.steps // 8 if args.decode_steps is None else args.decode_steps
    decode = []
    if decode_steps > 0:
        for qt, name, variant, kern in ((0, "q4_0", pkg.INPUT_REFERENCE, "gemv_q4_0_pairs_kernel"),
                                        (1, "q4_K", pkg.INPUT_REFERENCE, "gemv_q4_K_staged_kernel"),
                                        (2, "iq2_xxs", pkg.INPUT_BASELINE, "gemv_iq2_xxs_staged_kernel")):
            act_t = "q8_0" if qt == 0 else "q8_K"
            for dm in (8, 16):
                # from M = 9 at K = 4096 all three formats run the MFMA tile kernels
                kname = {(0, 16): "gemv_q4_0_mfma_kernel<16, 16>", (1, 16): "gemv_q4_K_mfma_kernel<16>",
                         (2, 16): "gemv_iq2_xxs_mfma_kernel<16>"}.get((qt, dm), f"{kern}<{dm}>")
                decode.append(gemv_item(torch, pkg, f"m{dm}_{name}: {name} x {act_t} GEMV M={dm} N=4096 K=4096, "
                                        "32 rotating weight copies", qt, dm, 4096, 4096, decode_steps,
                                        max(decode_steps // 10, 32), variant, kname))

    cpu = cpu_baseline(args.cpu_seconds) if args.cpu_seconds > 0 else None
    if cpu:
        log(f"[bench] cpu baseline: {cpu}")

    items = [x for x in (gemm, q4k, iq2, prefill, *gemv_kq, *decode) if x is not None]
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / steps, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded mt19937 U[-1,1) weights quantized to q4_0, activations to q8_0)",
        "config": {"workload": "c1: q4_0 x q8_0 GEMV M=1 N=4096 K=4096, 32 rotating weight copies (302 MB)",
                   "m": m, "n": n, "k": k, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_for("gemv_q4_0_m1_kernel", "c1"),
                     "kernel": "gemv_q4_0_m1_kernel", "kernel_us": round(kernel_us, 4),
                     "bytes_per_launch": per_call},
        "e2e_with_quantize_gbs": round(e2e_gbs, 2),
        "verify": ver1,
        "gemm": gemm,
        "q4_K": q4k,
        "iq2_xxs": iq2,
        "prefill": prefill,
        "gemv_q4_K": gemv_kq[0],
        "gemv_iq2_xxs": gemv_kq[1],
        "decode": decode,
        "verified": bool(ver1["passed"] and all(x["verify"]["passed"] for x in items)),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
