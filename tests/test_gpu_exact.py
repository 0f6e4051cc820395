"""GPU bit-exactness of every product kernel on exact-arithmetic inputs.

On the inputs of tests/exact_inputs.py (power-of-two scales, magnitudes
bounded so that every partial sum is an integer multiple of one unit below
2**24) every fp32 step is exact, so the output does not depend on the
summation order: each kernel must equal the oracle (the reference's order,
llama_reference.cpp:113-161) bit for bit. An integer block sum that is off by
one changes the output (tests/test_exact_inputs.py shows it on the CPU), so
this pins the integer part of every GEMV kernel, which the 1e-5 * sum|terms|
tolerance of the other tests cannot.

The shapes follow the kernel selection of launch_gemv (csrc/gemv.hip) and
launch_kquant_gemv (csrc/gemv_kquant.hip), named per case; PATH_GEMV is asked
for explicitly, so a shape that stopped taking the GEMV fails instead of
silently running another kernel.
"""
from __future__ import annotations

import numpy as np
import pytest

from exact_inputs import exact_case

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def dev(torch, arr):
    if arr.dtype == np.float32:
        return torch.from_numpy(np.ascontiguousarray(arr)).cuda()
    b = np.ascontiguousarray(arr).view(np.uint8).reshape(arr.shape[0], -1)
    return torch.from_numpy(b).cuda()


def assert_bits_equal(got, expect, label):
    g = np.ascontiguousarray(got, dtype=np.float32).view(np.uint32)
    e = np.ascontiguousarray(expect, dtype=np.float32).view(np.uint32)
    bad = np.flatnonzero(g != e)
    assert bad.size == 0, (f"{label}: {bad.size} outputs differ, first at {np.unravel_index(bad[0], g.shape)}: "
                           f"got {got.flat[bad[0]]!r} expected {expect.flat[bad[0]]!r}")


# (qtype, m, n, k, kernel the GEMV dispatch picks)
GEMV_CASES = [
    (0, 1, 4096, 4096, "gemv_q4_0_m1_kernel<true> (c1)"),
    (0, 1, 77, 320, "gemv_q4_0_m1_kernel<true>, dword tail"),
    (0, 1, 64, 65536, "gemv_q4_0_m1_kernel<false> (row past 64 KB of LDS)"),
    (0, 1, 100, 8192, "gemv_q4_0_m1_kernel<true>, k = 8192"),
    (0, 2, 4096, 4096, "gemv_q4_0_pairs_kernel<2>"),
    (0, 5, 300, 4096, "gemv_q4_0_pairs_kernel<5>"),
    (0, 3, 256, 1536, "gemv_q4_0_pairs_kernel<3>, k = 1536"),
    (0, 9, 77, 320, "gemv_q4_0_pairs_kernel<9> (k % 256 != 0)"),
    (0, 2, 64, 65536, "gemv_q4_0_pairs_kernel<2>, k = 65536"),
    (0, 3, 64, 65536, "gemv_q4_0_kernel<3> (8-block groups)"),
    (0, 4, 40, 65536, "gemv_q4_0_kernel<4> (8-block groups)"),
    (0, 6, 300, 4096, "gemv_q4_0_mfma_chunk_kernel<1>"),
    (0, 16, 300, 4096, "gemv_q4_0_mfma_chunk_kernel<1>"),
    (0, 4, 256, 1536, "gemv_q4_0_mfma_chunk_kernel<1>, idle waves"),
    (0, 17, 300, 4096, "gemv_q4_0_mfma_chunk_kernel<2>"),
    (0, 65, 130, 4096, "gemv_q4_0_mfma_chunk_kernel<5>"),
    (0, 128, 256, 4096, "gemv_q4_0_mfma_chunk_kernel<8>"),
    (0, 5, 100, 8192, "gemv_q4_0_mfma_chunk_kernel<1>, 2 rounds"),
    (0, 33, 100, 8192, "gemv_q4_0_mfma_chunk_kernel<3>, 2 rounds"),
    (0, 128, 64, 14336, "gemv_q4_0_mfma_chunk_kernel<8>, 3.5 rounds"),
    (1, 1, 4096, 4096, "gemv_q4_K_kernel<1, true> (activation row in LDS)"),
    (1, 1, 64, 65536, "gemv_q4_K_kernel<1> (row past 64 KB of LDS)"),
    (1, 2, 4096, 4096, "gemv_q4_K_staged_kernel<2>"),
    (1, 4, 300, 4096, "gemv_q4_K_staged_kernel<4>"),
    (1, 9, 100, 1536, "gemv_q4_K_staged_kernel<9> (k % 1024 != 0)"),
    (1, 16, 100, 1536, "gemv_q4_K_staged_kernel<16>"),
    (1, 4, 64, 32768, "gemv_q4_K_kernel<4> (rows too long to stage)"),
    (1, 5, 300, 4096, "gemv_q4_K_mfma_chunk_kernel<1>"),
    (1, 16, 300, 4096, "gemv_q4_K_mfma_chunk_kernel<1>"),
    (1, 17, 300, 4096, "gemv_q4_K_mfma_chunk_kernel<2>"),
    (1, 128, 256, 4096, "gemv_q4_K_mfma_chunk_kernel<8>"),
    (1, 5, 100, 8192, "gemv_q4_K_mfma_chunk_kernel<1>, 2 rounds"),
    (1, 40, 64, 14336, "gemv_q4_K_mfma_chunk_kernel<3>, 3.5 rounds"),
    (2, 1, 4096, 4096, "gemv_iq2_xxs_kernel<1>"),
    (2, 1, 300, 2560, "gemv_iq2_xxs_kernel<1>, a partial second step"),
    (2, 1, 100, 1792, "gemv_iq2_xxs_kernel<1>, one partial step"),
    (2, 1, 64, 65536, "gemv_iq2_xxs_kernel<1>, 32 steps"),
    (2, 2, 4096, 4096, "gemv_iq2_xxs_staged_kernel<2>"),
    (2, 4, 300, 4096, "gemv_iq2_xxs_staged_kernel<4>"),
    (2, 9, 100, 1536, "gemv_iq2_xxs_staged_kernel<9> (k % 2048 != 0)"),
    (2, 3, 64, 65536, "gemv_iq2_xxs_kernel<3> (rows too long to stage)"),
    (2, 5, 300, 4096, "gemv_iq2_xxs_mfma_sb_kernel<5> (two-half copies)"),
    (2, 8, 300, 4096, "gemv_iq2_xxs_mfma_sb_kernel<8>"),
    (2, 9, 300, 4096, "gemv_iq2_xxs_mfma_chunk_kernel<1>"),
    (2, 16, 300, 4096, "gemv_iq2_xxs_mfma_chunk_kernel<1>"),
    (2, 17, 300, 4096, "gemv_iq2_xxs_mfma_chunk_kernel<2>"),
    (2, 128, 256, 4096, "gemv_iq2_xxs_mfma_chunk_kernel<8>"),
    (2, 5, 100, 8192, "gemv_iq2_xxs_mfma_chunk_kernel<1>, 2 rounds"),
    (2, 70, 40, 8192, "gemv_iq2_xxs_mfma_chunk_kernel<5>, 2 rounds"),
]


@pytest.mark.parametrize("qtype,m,n,k,kernel", GEMV_CASES, ids=[f"{c[0]}-{c[1]}x{c[2]}x{c[3]}" for c in GEMV_CASES])
def test_gemv_bit_exact(hip, torch_gpu, oracle, qtype, m, n, k, kernel):
    torch = torch_gpu
    say(f"exact gemv type={qtype} {m}x{n}x{k}: {kernel}")
    x, aq, w, r, _ = exact_case(oracle, qtype, m, n, k, seed=m * 1009 + n + k + qtype)
    expect = oracle.matmul(qtype, w, aq, m, n, k)
    got = hip.mul_mat(qtype, dev(torch, w), dev(torch, aq), m, n, k, path=hip.PATH_GEMV)
    torch.cuda.synchronize()
    assert_bits_equal(got.cpu().numpy(), expect, f"{kernel} (|a| <= {r})")


# pfng_hip_compute: the fused quantize + GEMV kernels (q4_0 m <= 2, the
# K-quants at m == 1) and the separate quantize + product beyond
COMPUTE_CASES = [
    (0, 1, 4096, 4096, "gemv_q4_0_fused_kernel<1>"),
    (0, 2, 4096, 4096, "gemv_q4_0_fused_kernel<2>"),
    (0, 1, 300, 1984, "gemv_q4_0_fused_kernel<1>, k % 256 != 0"),
    (1, 1, 4096, 4096, "gemv_q4_K_kernel<1, true, true> (fused)"),
    (2, 1, 4096, 4096, "gemv_iq2_xxs_fused_kernel"),
    (0, 24, 200, 4096, "quantize_q8_0 + chunked GEMV"),
    (1, 9, 200, 4096, "quantize_q8_K + chunked GEMV"),
    (2, 480, 256, 1536, "quantize_q8_K + GEMM"),
]


@pytest.mark.parametrize("qtype,m,n,k,kernel", COMPUTE_CASES,
                         ids=[f"{c[0]}-{c[1]}x{c[2]}x{c[3]}" for c in COMPUTE_CASES])
def test_compute_bit_exact(hip, torch_gpu, oracle, qtype, m, n, k, kernel):
    torch = torch_gpu
    say(f"exact compute type={qtype} {m}x{n}x{k}: {kernel}")
    x, aq, w, r, _ = exact_case(oracle, qtype, m, n, k, seed=m * 13 + n + k + qtype)
    expect = oracle.compute(qtype, x, w)
    got = hip.compute(qtype, dev(torch, x), dev(torch, w), n)
    torch.cuda.synchronize()
    assert_bits_equal(got.cpu().numpy(), expect, f"{kernel} (|a| <= {r})")


# The MFMA GEMMs: their block sums are also pinned by pfng_hip_block_isums;
# here the whole product including the fp32 epilogue, on the tile plans the
# shapes select (c0's whole-K 32x96 tile, the 128x128 tile at c4, the 32x32
# tiles, the K-quant slices at c2 and c3). At c3 and c4 the oracle takes 32
# sampled rows.
GEMM_CASES = [
    (0, 480, 1536, 1536, None),
    (0, 2048, 11008, 4096, 32),
    (0, 64, 100, 2048, None),
    (0, 100, 77, 256, None),
    (0, 200, 3072, 2048, 32),
    (1, 480, 1536, 1536, None),
    (1, 470, 1500, 1536, None),
    (1, 300, 2000, 1024, None),
    (1, 130, 65, 768, None),
    (1, 2048, 1024, 256, None),
    (2, 512, 4096, 4096, 32),
    (2, 96, 130, 1024, None),
    (2, 2048, 2048, 256, 64),
]


@pytest.mark.parametrize("qtype,m,n,k,sample", GEMM_CASES, ids=[f"{c[0]}-{c[1]}x{c[2]}x{c[3]}" for c in GEMM_CASES])
def test_mfma_bit_exact(hip, torch_gpu, oracle, qtype, m, n, k, sample):
    torch = torch_gpu
    say(f"exact mfma type={qtype} {m}x{n}x{k}")
    x, aq, w, r, _ = exact_case(oracle, qtype, m, n, k, seed=m + n + k + qtype)
    got = hip.mul_mat(qtype, dev(torch, w), dev(torch, aq), m, n, k, path=hip.PATH_MFMA)
    torch.cuda.synchronize()
    rows = np.arange(m) if sample is None else np.sort(np.random.default_rng(m).choice(m, sample, replace=False))
    expect = oracle.matmul(qtype, w, np.ascontiguousarray(aq[rows]), len(rows), n, k)
    assert_bits_equal(got.cpu().numpy()[rows], expect, f"mfma type={qtype} {m}x{n}x{k} (|a| <= {r})")
