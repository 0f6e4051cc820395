"""Writes the golden fixtures under tests/golden/ from the reference's own code.

Run in the build container (where /root/reference exists):
    python tests/golden/make_fixtures.py

Sources:
  * oracle/_ref/libpfng_ref.so — the reference's bench/llama_reference/llama_reference.cpp
    and bench/framework/benchmark.cpp compiled unmodified by oracle/Makefile; its
    create_input (std::mt19937, seed 1, benchmark.cpp:34-94), quantize_row_* and compute.
  * kernels/iq2_xxs-q8_K-RVV-common/ggml_min.h:58-134 read as text for the IQ2_XXS
    grid and sign tables (data values only).

Outputs (data only — inputs and the reference's outputs):
  ref_vectors.npz   seeded inputs, quantized activations and compute() outputs
  ref_quant_edges.npz  crafted quantizer inputs with the reference's block bytes
  iq2xxs_tables.json   the 256-entry grid and 128-entry sign table
"""
from __future__ import annotations

import json
import os
import re
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

import oracle as O  # noqa: E402

REF_ROOT = os.environ.get("PFNG_REFERENCE", "/root/reference")

# (type, m, n, k): small seeded cases; (24, 32, 256) is the shape of the
# reference's recorded preflight (kernels/q4_0-q8_0-IME-m4i/.../performance.md:63-65)
CASES = [(O.Q4_0, 24, 32, 256), (O.Q4_0, 3, 5, 96), (O.Q4_K, 8, 16, 512), (O.IQ2_XXS, 8, 16, 512)]


def edge_inputs(k: int) -> np.ndarray:
    rng = np.random.default_rng(7)
    rows = []
    rows.append(np.zeros(k, np.float32))                                   # all zero -> d = 0
    r = rng.uniform(-1, 1, k).astype(np.float32); r[5] = -3.0; rows.append(r)  # negative extreme
    rows.append((np.arange(k, dtype=np.float32) - k / 2) * np.float32(0.5))  # exact ties at .5 steps
    rows.append(rng.uniform(-1e-6, 1e-6, k).astype(np.float32))            # tiny values, subnormal fp16 d
    rows.append(rng.uniform(-6e4, 6e4, k).astype(np.float32))              # near fp16 max
    rows.append(np.full(k, 0.75, np.float32))                             # constant block
    r = rng.standard_normal(k).astype(np.float32) * 3; rows.append(r)       # gaussian
    r = np.zeros(k, np.float32); r[::17] = 1.0; rows.append(r)              # sparse
    return np.stack(rows)


def main() -> None:
    O.build(ref=True)
    R = O.ref()
    vec = {}
    for (t, m, n, k) in CASES:
        tag = f"{O.TYPE_NAMES[t]}_{m}x{n}x{k}"
        act = np.empty((m, k), np.float32)
        w = np.zeros((n, k // O.QK[t]), O.WEIGHT_DTYPE[t])
        assert R.ref_create_input(t, 1, m, n, k, O._ptr(act), O._ptr(w)) == 0
        aq = np.zeros((m, k // O.QK[t]), O.ACT_DTYPE[t])
        qfn = R.ref_quantize_row_q8_0 if t == O.Q4_0 else R.ref_quantize_row_q8_K
        for r in range(m):
            qfn(O._ptr(act[r]), O._ptr(aq[r]), k)
        out = np.zeros((m, n), np.float32)
        assert R.ref_compute(t, O._ptr(act), O._ptr(w), O._ptr(out), m, n, k) == 0
        vec[f"{tag}/act"] = act
        vec[f"{tag}/weight"] = w.view(np.uint8)
        vec[f"{tag}/act_q"] = aq.view(np.uint8)
        vec[f"{tag}/out"] = out
    np.savez_compressed(os.path.join(HERE, "ref_vectors.npz"), **vec)

    edges = {}
    for name, k, fn, dt in [("q8_0", 64, R.ref_quantize_row_q8_0, O.DT_Q8_0),
                            ("q8_K", 256, R.ref_quantize_row_q8_K, O.DT_Q8_K),
                            ("q4_0", 64, R.ref_quantize_row_q4_0, O.DT_Q4_0),
                            ("q4_K", 256, R.ref_quantize_row_q4_K, O.DT_Q4_K)]:
        x = edge_inputs(k)
        y = np.zeros((x.shape[0], k // (32 if name in ("q8_0", "q4_0") else 256)), dt)
        for r in range(x.shape[0]):
            fn(O._ptr(x[r]), O._ptr(y[r]), k)
        edges[f"{name}/x"] = x
        edges[f"{name}/y"] = y.view(np.uint8)
    specials = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65520.0, 1e9, 6.1035156e-05, 5.9604645e-08, 2.9802322e-08,
                         1e-10, 0.1, 1.0 / 3.0, 2049.0, 2051.0, np.inf, -np.inf, np.nan], np.float32)
    edges["fp16/x"] = specials
    edges["fp16/y"] = np.array([R.ref_fp32_to_fp16(float(v)) for v in specials], np.uint16)
    np.savez_compressed(os.path.join(HERE, "ref_quant_edges.npz"), **edges)

    src = open(os.path.join(REF_ROOT, "kernels/iq2_xxs-q8_K-RVV-common/ggml_min.h")).read()
    grid = [int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", src.split("iq2xxs_grid[256] = {")[1].split("};")[0])]
    signs = [int(v) for v in re.findall(r"\d+", src.split("ksigns_iq2xs[128] = {")[1].split("};")[0])]
    small = open(os.path.join(REF_ROOT, "kernels/common/iq2_xxs.h")).read()
    grid32 = [int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", small.split("grid = {")[1].split("};")[0])]
    assert len(grid) == 256 and len(signs) == 128 and len(grid32) == 32
    with open(os.path.join(HERE, "iq2xxs_tables.json"), "w") as f:
        json.dump({"source": "kernels/iq2_xxs-q8_K-RVV-common/ggml_min.h:58-134, kernels/common/iq2_xxs.h:14-23",
                   "iq2xxs_grid": [f"0x{v:016x}" for v in grid], "ksigns_iq2xs": signs,
                   "reduced_grid_32": [f"0x{v:016x}" for v in grid32]}, f, indent=1)
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
