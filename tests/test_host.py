"""Host side of the product: the input generator and weight quantizers behind
pfng_host_create_input (mirror of bench/framework/benchmark.cpp:29-94) and the
C++ harness binary (mirror of bench/main.cpp). CPU tests compare the product's
bytes with the oracle's (which the oracle tests pin to the reference build and
its fixtures); GPU tests drive pfng_bench end to end."""
from __future__ import annotations

import os
import re
import subprocess

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(REPO, "qgemm-perf-framework-ng_amd", "pfng_bench")


@pytest.mark.parametrize("qtype", [0, 1, 2])
@pytest.mark.parametrize("variant", [0, 1])
@pytest.mark.parametrize("m,n,k", [(3, 5, 256), (24, 32, 256), (1, 7, 1024)])
def test_create_input_matches_oracle(pkg, oracle, qtype, variant, m, n, k):
    act, w = pkg.create_input(qtype, m, n, k, seed=1 + m, variant=variant)
    act_o, w_o = oracle.create_input(qtype, m, n, k, seed=1 + m, variant=variant)
    assert np.array_equal(act.view(np.uint32), act_o.view(np.uint32))
    assert np.array_equal(w.reshape(-1), np.ascontiguousarray(w_o).view(np.uint8).reshape(-1))


def test_create_input_rejects_bad_k(pkg):
    with pytest.raises(ValueError):
        pkg.create_input(0, 1, 1, 48)
    with pytest.raises(ValueError):
        pkg.create_input(2, 1, 1, 128)


@pytest.mark.parametrize("qtype", [0, 1])
def test_quantize_weights_matches_oracle(pkg, oracle, qtype):
    rng = np.random.default_rng(qtype + 11)
    rows, k = 37, 1024
    x = (rng.standard_normal((rows, k)) * rng.uniform(1e-4, 30, (rows, 1))).astype(np.float32)
    x[0] = 0.0                                   # all-zero blocks
    x[1, :32] = 7.0                              # constant block
    x[2, :256] = np.linspace(-1, 1, 256)         # ties at x/d + 8.5
    x[3, ::2] = -x[3, 1::2]                      # signed maxima of both signs
    got = pkg.quantize_weights(qtype, x)
    expect = oracle.quantize_q4_0(x) if qtype == 0 else oracle.quantize_q4_K(x)
    assert np.array_equal(got.reshape(-1), expect.view(np.uint8).reshape(-1))


def test_fp16_conversions_match_oracle(pkg, oracle):
    L = pkg.lib()
    halves = np.arange(65536, dtype=np.uint16)
    finite = halves[(halves & 0x7C00) != 0x7C00]
    got = np.array([L.pfng_host_fp16_to_fp32(int(h)) for h in finite[::7]], np.float32)
    assert np.array_equal(got.view(np.uint32), oracle.fp16_to_fp32(finite[::7]).view(np.uint32))
    rng = np.random.default_rng(2)
    f = np.concatenate([rng.standard_normal(3000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 3000),
                        np.array([0.0, -0.0, 65504.0, 65520.0, 1e-8, 6.1e-5, 5.96e-8, np.inf, -np.inf], np.float32)])
    f = f.astype(np.float32)
    got = np.array([L.pfng_host_fp32_to_fp16(float(v)) for v in f], np.uint16)
    assert np.array_equal(got, oracle.fp32_to_fp16(f))


@pytest.mark.parametrize("qtype,variant", [(0, 0), (1, 0), (2, 0), (2, 1)])
@pytest.mark.parametrize("m,n,k", [(3, 5, 256), (24, 32, 512), (9, 17, 768)])
def test_host_compute_matches_oracle(pkg, oracle, qtype, variant, m, n, k):
    """The harness's verification reference (pfng_host_compute) is the oracle's
    compute() bit for bit, for one and for several threads (the oracle tests pin
    compute() to the reference build and its fixtures)."""
    if k % pkg.QK[qtype]:
        pytest.skip("k is not a multiple of the block")
    act, w = pkg.create_input(qtype, m, n, k, seed=7 + m, variant=variant)
    w_o = w.reshape(-1).view(oracle.WEIGHT_DTYPE[qtype]).reshape(n, -1)
    expect = oracle.compute(qtype, act, w_o)
    for threads in (1, 4):
        got = pkg.host_compute(qtype, act, w, n, threads=threads)
        assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))


def test_host_compute_rejects_bad_arguments(pkg):
    with pytest.raises(ValueError):
        pkg.host_compute(0, np.zeros((2, 48), np.float32), np.zeros((3, 27), np.uint8), 3)
    with pytest.raises(ValueError):
        pkg.host_compute(3, np.zeros((2, 64), np.float32), np.zeros((3, 36), np.uint8), 3)


def test_checksum_matches_oracle(pkg, oracle):
    x = np.random.default_rng(3).standard_normal((33, 97)).astype(np.float32)
    assert pkg.checksum(x) == oracle.checksum(x)


def run_bench(*args, timeout=120):
    return subprocess.run([BENCH, *args], capture_output=True, text=True, timeout=timeout)


def test_harness_lists_kernel_ids():
    r = run_bench("--list")
    assert r.returncode == 0, r.stderr
    ids = [line.split()[0] for line in r.stdout.splitlines() if line.strip()]
    assert {"q4_0-q8_0-HIP-mi355x", "q4_0-q8_0-HIP-gemv", "q4_0-q8_0-HIP-mfma", "q4_0-q8_0-HIP-naive",
            "q4_K-q8_K-HIP-mi355x", "q4_K-q8_K-HIP-naive", "iq2_xxs-q8_K-HIP-mi355x",
            "iq2_xxs-q8_K-HIP-naive"} <= set(ids)
    assert len(ids) == len(set(ids))


def test_harness_build_info_and_usage():
    r = run_bench("--build-info")
    assert r.returncode == 0 and "arch: gfx950" in r.stdout
    assert run_bench("--m", "0", "--n", "1", "--k", "32").returncode == 2
    assert run_bench("--bogus").returncode == 2
    assert run_bench("--input", "other").returncode == 2


def parse_report(text):
    """kernel id -> dict(status lines) from pfng_bench's report."""
    out, cur = {}, None
    for line in text.splitlines():
        m = re.match(r"^\[(\S+)\] ", line)
        if m:
            cur = out.setdefault(m.group(1), {})
            continue
        if cur is not None and ":" in line:
            key, val = line.split(":", 1)
            cur[key.strip()] = val.strip()
    return out


@pytest.mark.gpu
def test_harness_runs_every_kernel_id_with_verification(hip):
    print("[case] pfng_bench --kernel all 24x32x256", flush=True)
    r = run_bench("--kernel", "all", "--m", "24", "--n", "32", "--k", "256", "--samples", "3", "--warmup", "1",
                  "--input", "reference", timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    rep = parse_report(r.stdout)
    assert len(rep) == 8
    # the GEMV ID declines M > 8 through validate(), as the reference's
    # adapters decline shapes they do not take
    assert rep["q4_0-q8_0-HIP-gemv"]["status"].startswith("SKIP")
    for kid, fields in rep.items():
        if kid == "q4_0-q8_0-HIP-gemv":
            continue
        assert fields.get("verify", "").startswith("PASS"), (kid, fields)
        assert "error elements" in fields and fields["error elements"].startswith("0/768"), (kid, fields)
    r4 = run_bench("--kernel", "q4_0-q8_0-HIP-gemv", "--m", "4", "--n", "32", "--k", "256", "--samples", "3",
                   "--warmup", "1", timeout=120)
    assert r4.returncode == 0, r4.stdout + r4.stderr
    assert parse_report(r4.stdout)["q4_0-q8_0-HIP-gemv"]["verify"].startswith("PASS")
    # the documented checksum of q4_0 24x32x256, seed 1
    # (kernels/q4_0-q8_0-IME-m4i/.../performance.md:65): 3.84864689
    cs = float(rep["q4_0-q8_0-HIP-naive"]["checksum"])
    assert abs(cs - 3.84864689) <= 3 * 1.90735e-6
    assert abs(float(rep["q4_0-q8_0-HIP-mi355x"]["checksum"]) - 3.84864689) <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("kid,m,n,k,variant", [
    ("q4_0-q8_0-HIP-mi355x", 480, 1536, 1536, "reference"),
    ("q4_0-q8_0-HIP-mi355x", 1, 4096, 4096, "reference"),
    ("q4_K-q8_K-HIP-mi355x", 480, 1536, 1536, "reference"),
    ("iq2_xxs-q8_K-HIP-mi355x", 512, 4096, 4096, "baseline"),
])
def test_harness_baseline_configs_verify(hip, kid, m, n, k, variant):
    print(f"[case] pfng_bench {kid} {m}x{n}x{k}", flush=True)
    r = run_bench("--kernel", kid, "--m", str(m), "--n", str(n), "--k", str(k), "--samples", "3", "--warmup", "2",
                  "--input", variant, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    fields = parse_report(r.stdout)[kid]
    assert fields["verify"].startswith("PASS") and fields["error elements"].startswith(f"0/{m * n}"), fields
