"""GPU parity: every HIP path through the C-ABI against the CPU oracle.

Bars: quantized activation bytes and integer block sums bit-exact; the naive
path's fp32 output bit-exact (it keeps the reference's operation order); the
GEMV and MFMA paths within |err| <= 1e-5 * sum|terms| per output element.
At the baseline configs' full sizes the oracle checks a seeded sample of rows.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-5  # the fp32 contract: |gpu - oracle| <= 1e-5 * sum|terms|


def say(msg):
    print(f"[case] {msg}", flush=True)


def dev(torch, arr):
    """numpy (structured) array -> CUDA uint8/float tensor with the same bytes."""
    if arr.dtype == np.float32:
        return torch.from_numpy(np.ascontiguousarray(arr)).cuda()
    b = np.ascontiguousarray(arr).view(np.uint8).reshape(arr.shape[0], -1)
    return torch.from_numpy(b).cuda()


def host_blocks(t, dtype):
    b = t.cpu().numpy()
    return b.reshape(-1).view(dtype).reshape(b.shape[0], -1)


def doubled_scales(w):
    """Copy of weight blocks with every fp16 `d` (and q4_K's `dmin`) multiplied
    by 2 exactly (the exponent field raised by one; all scales here are normal
    and far from the fp16 maximum). Every output of a correct product doubles
    exactly."""
    w2 = w.copy()
    for field in ("d", "dmin"):
        if field not in w2.dtype.names:
            continue
        bits = w2[field].view(np.uint16)
        exp = (bits >> 10) & 0x1F
        assert ((exp >= 1) & (exp <= 29)).all()
        w2[field] = (bits + np.uint16(1 << 10)).view(w2[field].dtype)
    return w2


def check_full_size_properties(hip, torch, qtype, w, wt, aq_t, got, m, n, k):
    """Size-independent checks on a whole output: permuting weight rows
    permutes output columns bit for bit (each column's arithmetic is independent
    of its tile), and doubling every weight scale doubles every output exactly."""
    permn = torch.randperm(n, generator=torch.Generator().manual_seed(1)).cuda()
    got_n = hip.mul_mat(qtype, wt[permn].contiguous(), aq_t, m, n, k)
    torch.cuda.synchronize()
    assert torch.equal(got_n, got[:, permn])
    del got_n
    got_2 = hip.mul_mat(qtype, dev(torch, doubled_scales(w)), aq_t, m, n, k)
    torch.cuda.synchronize()
    assert torch.equal(got_2, got * 2)


def run_mul_mat(hip, torch, qtype, w, aq, m, n, k, path):
    out = hip.mul_mat(qtype, dev(torch, w), dev(torch, aq), m, n, k, path=path)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check_close(oracle, qtype, got, w, aq, m, n, k, rows=None, label=""):
    """Compare got (rows x n) with the oracle on activation rows `rows`."""
    if rows is None:
        rows = np.arange(m)
    sub = np.ascontiguousarray(aq[rows])
    expect = oracle.matmul(qtype, w, sub, len(rows), n, k)
    terms = oracle.abs_terms(qtype, w, sub, len(rows), n, k)
    ok, worst, idx = oracle.within_tolerance(got[rows], expect, terms, TOL)
    assert ok, f"{label}: worst err/bound {worst:.3g} at {np.unravel_index(idx, expect.shape)}"
    return worst


# ------------------------------------------------------------ quantizers ----

@pytest.mark.parametrize("rows,k", [(1, 32), (37, 4096), (480, 1536), (3, 96)])
def test_quantize_q8_0_bit_exact(hip, torch_gpu, oracle, rows, k):
    torch = torch_gpu
    say(f"quantize_q8_0 rows={rows} k={k}")
    rng = np.random.default_rng(rows * 7 + k)
    x = (rng.standard_normal((rows, k)) * rng.uniform(1e-3, 50, (rows, 1))).astype(np.float32)
    x[0, :min(k, 32)] = 0.0                      # a zero block
    x[-1, :8] = np.float32(0.5) * np.arange(8)   # ties
    got = hip.quantize_q8_0(dev(torch, x))
    torch.cuda.synchronize()
    expect = oracle.quantize_q8_0(x)
    assert np.array_equal(got.cpu().numpy().reshape(-1), expect.view(np.uint8).reshape(-1))


@pytest.mark.parametrize("rows,k", [(1, 256), (29, 4096), (512, 4096)])
def test_quantize_q8_K_bit_exact(hip, torch_gpu, oracle, rows, k):
    torch = torch_gpu
    say(f"quantize_q8_K rows={rows} k={k}")
    rng = np.random.default_rng(rows * 5 + k)
    x = (rng.standard_normal((rows, k)) * rng.uniform(1e-3, 50, (rows, 1))).astype(np.float32)
    x[0, :256] = 0.0
    got = hip.quantize_q8_K(dev(torch, x))
    torch.cuda.synchronize()
    expect = oracle.quantize_q8_K(x)
    assert np.array_equal(got.cpu().numpy().reshape(-1), expect.view(np.uint8).reshape(-1))


@pytest.mark.parametrize("name,rows,k", [("q8_0", 3, 1280), ("q8_0", 1, 64), ("q8_K", 3, 1280), ("q8_K", 5, 4096)])
@pytest.mark.parametrize("offset", [2, 4, 16])
def test_quantize_output_alignment(hip, torch_gpu, oracle, name, rows, k, offset):
    """Both store paths: a dword-aligned output is assembled in LDS and written
    through as dwords (offsets 4 and 16), a q8_0 output at an odd half-word is
    stored in 16-bit pieces (offset 2; q8_K outputs must be 4-byte aligned, and
    the library rejects one at offset 2 before launching anything). Ragged
    shapes leave the last workgroup partly empty; the bytes around the output
    must stay untouched."""
    torch = torch_gpu
    say(f"quantize {name} rows={rows} k={k} output offset {offset}")
    rng = np.random.default_rng(rows * 11 + k + offset)
    x = (rng.standard_normal((rows, k)) * rng.uniform(1e-3, 50, (rows, 1))).astype(np.float32)
    fn, ref = (hip.quantize_q8_0, oracle.quantize_q8_0) if name == "q8_0" else (hip.quantize_q8_K, oracle.quantize_q8_K)
    nbytes = rows * (k // 32) * 34 if name == "q8_0" else rows * (k // 256) * 292
    buf = torch.full((nbytes + 64,), 0xA5, dtype=torch.uint8, device="cuda")
    if name == "q8_K" and offset % 4:
        with pytest.raises(RuntimeError, match="4-byte aligned"):
            fn(dev(torch, x), out=buf[offset:offset + nbytes])
        return
    fn(dev(torch, x), out=buf[offset:offset + nbytes])
    torch.cuda.synchronize()
    got = buf.cpu().numpy()
    assert np.array_equal(got[offset:offset + nbytes], ref(x).view(np.uint8).reshape(-1))
    assert (got[:offset] == 0xA5).all() and (got[offset + nbytes:] == 0xA5).all(), "bytes outside the output written"


@pytest.mark.parametrize("name", ["q8_0", "q8_K"])
def test_quantizer_edges_match_reference_fixture(hip, torch_gpu, name):
    torch = torch_gpu
    say(f"quantize edges {name}")
    e = np.load(os.path.join(GOLDEN, "ref_quant_edges.npz"))
    x, y = e[f"{name}/x"], e[f"{name}/y"]
    fn = hip.quantize_q8_0 if name == "q8_0" else hip.quantize_q8_K
    got = fn(dev(torch, x))
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy().reshape(-1), y.reshape(-1))


# ------------------------------------------------- golden reference vectors ----

@pytest.mark.parametrize("tag,qtype", [("q4_0_24x32x256", 0), ("q4_0_3x5x96", 0), ("q4_K_8x16x512", 1),
                                       ("iq2_xxs_8x16x512", 2)])
def test_compute_matches_reference_vectors(hip, torch_gpu, oracle, tag, qtype):
    """pfng_hip_compute (GPU quantize + product) on the reference's own seeded inputs."""
    torch = torch_gpu
    say(f"compute golden {tag}")
    v = np.load(os.path.join(GOLDEN, "ref_vectors.npz"))
    act, w8, out_ref = v[f"{tag}/act"], v[f"{tag}/weight"], v[f"{tag}/out"]
    m, k = act.shape
    n = out_ref.shape[1]
    wt = torch.from_numpy(w8.reshape(n, -1)).cuda()
    # naive path: the reference's exact fp32 order -> bit-identical
    got = hip.compute(qtype, dev(torch, act), wt, n, path=hip.PATH_NAIVE)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy().view(np.uint32), out_ref.view(np.uint32))
    # automatic path: within tolerance, or declined (no tiled path takes the shape)
    if hip.auto_path(qtype, m, n, k) < 0:
        with pytest.raises(hip.PfngError) as e:
            hip.compute(qtype, dev(torch, act), wt, n, path=hip.PATH_AUTO)
        assert e.value.status == hip.ERR_UNSUPPORTED and "PFNG_PATH_NAIVE" in str(e.value)
        return
    got = hip.compute(qtype, dev(torch, act), wt, n, path=hip.PATH_AUTO)
    torch.cuda.synchronize()
    w = w8.reshape(-1).view(oracle.WEIGHT_DTYPE[qtype]).reshape(n, -1)
    aq = oracle.quantize_activation(qtype, act)
    check_close(oracle, qtype, got.cpu().numpy(), w, aq, m, n, k, label=tag)


# ------------------------------------------------------------------ naive ----

@pytest.mark.parametrize("qtype,m,n,k", [(0, 7, 33, 320), (1, 5, 9, 768), (2, 5, 9, 768)])
def test_naive_bit_exact(hip, torch_gpu, oracle, qtype, m, n, k):
    torch = torch_gpu
    say(f"naive type={qtype} {m}x{n}x{k}")
    act, w = oracle.create_input(qtype, m, n, k, seed=21)
    aq = oracle.quantize_activation(qtype, act)
    got = run_mul_mat(hip, torch, qtype, w, aq, m, n, k, hip.PATH_NAIVE)
    expect = oracle.matmul(qtype, w, aq, m, n, k)
    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))


# ------------------------------------------------------------------- GEMV ----

@pytest.mark.parametrize("m", [1, 2, 3, 5, 7, 8, 9, 12, 13, 15, 16])
@pytest.mark.parametrize("n,k", [(4096, 4096), (257, 1536), (64, 256), (33, 8192), (40, 65536), (129, 7680),
                                 (77, 320), (50, 64), (21, 20480), (37, 6144), (48, 2048), (100, 4096)])
def test_gemv_q4_0(hip, torch_gpu, oracle, m, n, k):
    """m = 1 (block pair per lane; the activation row copied into LDS in
    rounds of 16 KB up to 64 KB, k = 20480 taking two rounds, a dword tail at
    k = 320 and 64), m = 2..16 with the activations staged in LDS
    (m * (k / 64) * 76 + 16 <= 160 KB), m = 2..8 beyond that (groups of 8
    blocks per lane); at k % 256 == 0 from k = 512 the one-chunk 16x16 MFMA
    tile kernel, from m = 3..6 by k (k = 1536 and 2048 from m = 4, k = 4096
    from 6, above from 5), over up to 16 rounds (k = 1536 and 2048: waves
    without a K group; 6144 and 7680: waves with different numbers of rounds;
    100, 33, 37 and 129 columns partial tiles)."""
    torch = torch_gpu
    tiles = k % 256 == 0 and k >= 512
    if m > 8 and not tiles and m * (k // 64) * 76 + 16 > 160 * 1024:
        pytest.skip("m > 8 takes the GEMV below the tiles' k only while the staged activations fit in LDS")
    say(f"gemv q4_0 m={m} n={n} k={k}")
    act, w = oracle.create_input(0, m, n, k, seed=m * 31 + n)
    aq = oracle.quantize_q8_0(act)
    got = run_mul_mat(hip, torch, 0, w, aq, m, n, k, hip.PATH_GEMV)
    check_close(oracle, 0, got, w, aq, m, n, k, label=f"gemv m={m} n={n} k={k}")


@pytest.mark.parametrize("m", [17, 20, 31, 32, 33, 47, 48, 49, 63, 64, 65, 96, 127, 128])
@pytest.mark.parametrize("n", [4096, 37, 1])
def test_gemv_q4_0_chunked(hip, torch_gpu, oracle, m, n):
    """k = 4096, m = 17..128: the 16-row MFMA tile over chunks of 16 activation
    rows (each chunk's halves refilled while the other half is multiplied), a
    partial last chunk and tile; the generator's inputs, then random weight
    bytes against activations at the int8 limits."""
    torch = torch_gpu
    k = 4096
    say(f"gemv q4_0 chunked m={m} n={n}")
    act, w = oracle.create_input(0, m, n, k, seed=m * 13 + n)
    aq = oracle.quantize_q8_0(act)
    got = run_mul_mat(hip, torch, 0, w, aq, m, n, k, hip.PATH_GEMV)
    check_close(oracle, 0, got, w, aq, m, n, k, label=f"gemv chunked m={m} n={n}")
    wr = random_weight_blocks(oracle, 0, n, k, seed=71 + m)
    ax = oracle.quantize_q8_0(np.where(np.random.default_rng(m).random((m, k)) < 0.5, -1.0, 1.0).astype(np.float32))
    got = run_mul_mat(hip, torch, 0, wr, ax, m, n, k, hip.PATH_GEMV)
    check_close(oracle, 0, got, wr, ax, m, n, k, label=f"gemv chunked random bytes m={m} n={n}")


# ------------------------------------------------------------------- MFMA ----

@pytest.mark.parametrize("m,n,k", [(32, 32, 128), (100, 77, 256), (480, 1536, 1536), (9, 300, 640), (2048, 4096, 256),
                                   (1, 50, 128), (16, 4096, 4096), (33, 1000, 512), (64, 100, 2048), (65, 70, 256),
                                   (256, 4096, 4096), (470, 1500, 1536), (256, 1536, 1024), (300, 2000, 1024)])
def test_mfma_q4_0(hip, torch_gpu, oracle, m, n, k):
    torch = torch_gpu
    say(f"mfma q4_0 {m}x{n}x{k}")
    act, w = oracle.create_input(0, m, n, k, seed=m + n + k)
    aq = oracle.quantize_q8_0(act)
    got = run_mul_mat(hip, torch, 0, w, aq, m, n, k, hip.PATH_MFMA)
    rows = None if m * n * k <= 480 * 1536 * 1536 else np.sort(np.random.default_rng(1).choice(m, 64, replace=False))
    check_close(oracle, 0, got, w, aq, m, n, k, rows=rows, label=f"mfma {m}x{n}x{k}")


# block_isums runs the configuration the MFMA plan picks for the shape: 64x64
# with 2 waves (k % 256 != 0), 32x32 with 2 K-waves, 32x32 with 8 K-waves
# (decode batches, k % 1024 == 0), 64x64 with 4 waves (640x2048), 64x64 with
# 2 K-waves (200x3072x2048), whole-K 32x96 tiles (250x1540x1024, 470x1500x1536)
@pytest.mark.parametrize("m,n,k", [(32, 32, 128), (70, 45, 384), (64, 64, 1536), (9, 40, 256), (50, 33, 640),
                                   (96, 40, 512), (20, 50, 2048), (64, 33, 1024), (640, 2048, 256),
                                   (200, 3072, 2048), (250, 1540, 1024), (470, 1500, 1536)])
def test_block_isums_q4_0_bit_exact(hip, torch_gpu, oracle, m, n, k):
    torch = torch_gpu
    say(f"block isums q4_0 {m}x{n}x{k}")
    act, w = oracle.create_input(0, m, n, k, seed=5)
    aq = oracle.quantize_q8_0(act)
    got = hip.block_isums(0, dev(torch, w), dev(torch, aq), m, n, k)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), oracle.isums(0, w, aq, m, n, k))


# ---------------------------------------------------- full baseline configs ----

def test_config1_gemv_full_size(hip, torch_gpu, oracle):
    """c1: q4_0 GEMV M=1 N=4096 K=4096, whole output checked."""
    torch = torch_gpu
    say("c1 gemv 1x4096x4096")
    act, w = oracle.create_input(0, 1, 4096, 4096, seed=1)
    got = hip.compute(0, dev(torch, act), dev(torch, w), 4096)
    torch.cuda.synchronize()
    aq = oracle.quantize_q8_0(act)
    check_close(oracle, 0, got.cpu().numpy(), w, aq, 1, 4096, 4096, label="c1")


def test_config4_prefill_full_size_sampled(hip, torch_gpu, oracle):
    """c4: q4_0 GEMM M=2048 N=11008 K=4096; oracle on 24 seeded rows plus
    size-independent checks on the whole output (finite, activation-row and
    weight-row permutation equivariance, exact doubling with the weight scales)."""
    torch = torch_gpu
    m, n, k = 2048, 11008, 4096
    say("c4 mfma 2048x11008x4096")
    act, w = oracle.create_input(0, m, n, k, seed=1)
    wt = dev(torch, w)
    at = dev(torch, act)
    aq_t = hip.quantize_q8_0(at)
    got = hip.mul_mat(0, wt, aq_t, m, n, k)
    torch.cuda.synchronize()
    aq = oracle.quantize_q8_0(act)
    assert np.array_equal(aq_t.cpu().numpy().reshape(-1), aq.view(np.uint8).reshape(-1))
    g = got.cpu().numpy()
    assert np.isfinite(g).all()
    rows = np.sort(np.random.default_rng(4).choice(m, 24, replace=False))
    check_close(oracle, 0, g, w, aq, m, n, k, rows=rows, label="c4")
    # permuting activation rows permutes output rows exactly (tiles see the same blocks)
    perm = torch.randperm(m, generator=torch.Generator().manual_seed(0)).cuda()
    got_p = hip.mul_mat(0, wt, aq_t[perm].contiguous(), m, n, k)
    torch.cuda.synchronize()
    assert torch.equal(got_p, got[perm])
    del got_p
    check_full_size_properties(hip, torch, 0, w, wt, aq_t, got, m, n, k)


# ------------------------------------------------- q4_K / iq2_xxs MFMA ----

def random_weight_blocks(oracle, qtype, n, k, seed):
    """Weights with uniformly random bytes (every 6-bit scale and min, every
    grid index, sign index and scale nibble) and sane fp16 super-block scales."""
    rng = np.random.default_rng(seed)
    dt = oracle.WEIGHT_DTYPE[qtype]
    nb = k // oracle.QK[qtype]
    raw = rng.integers(0, 256, n * nb * dt.itemsize, dtype=np.uint8)
    w = raw.view(dt).reshape(n, nb).copy()
    w["d"] = oracle.fp32_to_fp16(rng.uniform(1e-3, 1e-2, (n, nb)).astype(np.float32))
    if qtype == oracle.Q4_K:
        w["dmin"] = oracle.fp32_to_fp16(rng.uniform(1e-3, 1e-2, (n, nb)).astype(np.float32))
    return w


def extreme_activation(oracle, m, k, seed):
    """q8_K rows at the int8 limits: every value +-127 (bsums +-2032)."""
    rng = np.random.default_rng(seed)
    x = np.where(rng.random((m, k)) < 0.5, -1.0, 1.0).astype(np.float32)
    return oracle.quantize_q8_K(x)


# the configuration follows the plan: 32x32 tiles with 4/2/1 super-block
# slices (small shapes), 64x64 with 2 slices (480x1536), 128x64 with 2 slices
# (2048x1024; 1000x2048x768: ragged row tile, three super-blocks over two
# slices) and 128x64 (2048x2048; 1000x4096x512: ragged row tile, two
# super-blocks), so the activation rows' direct-to-LDS copies run with rows
# past m and with a slice that has no super-block in its last step
@pytest.mark.parametrize("qtype", [1, 2])
@pytest.mark.parametrize("m,n,k", [(32, 64, 256), (100, 77, 512), (1, 1, 256), (130, 65, 768), (480, 64, 1536),
                                   (480, 1536, 256), (2048, 1024, 256), (2048, 2048, 256), (1000, 2048, 768),
                                   (1000, 4096, 512)])
def test_block_isums_kquant_bit_exact(hip, torch_gpu, oracle, qtype, m, n, k):
    torch = torch_gpu
    say(f"block isums type={qtype} {m}x{n}x{k}")
    act, w = oracle.create_input(qtype, m, n, k, seed=m + 3 * n)
    aq = oracle.quantize_q8_K(act)
    got = hip.block_isums(qtype, dev(torch, w), dev(torch, aq), m, n, k)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), oracle.isums(qtype, w, aq, m, n, k))


@pytest.mark.parametrize("qtype", [1, 2])
@pytest.mark.parametrize("m,n,k", [(96, 130, 1024), (480, 1536, 512)])  # 32x32 with 4 slices; 64x64 with 2
def test_block_isums_kquant_random_bytes_and_extremes(hip, torch_gpu, oracle, qtype, m, n, k):
    torch = torch_gpu
    say(f"block isums random bytes type={qtype} {m}x{n}x{k}")
    w = random_weight_blocks(oracle, qtype, n, k, seed=17 + qtype)
    for aq in (oracle.quantize_q8_K(oracle.create_input(qtype, m, 1, k, seed=9)[0]),
               extreme_activation(oracle, m, k, seed=3)):
        got = hip.block_isums(qtype, dev(torch, w), dev(torch, aq), m, n, k)
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy(), oracle.isums(qtype, w, aq, m, n, k))
        out = run_mul_mat(hip, torch, qtype, w, aq, m, n, k, hip.PATH_MFMA)
        check_close(oracle, qtype, out, w, aq, m, n, k, label=f"random bytes type={qtype}")


@pytest.mark.parametrize("qtype", [1, 2])
@pytest.mark.parametrize("m,n,k", [(32, 64, 256), (100, 77, 512), (1, 300, 768), (9, 1, 256), (257, 129, 1280)])
def test_mfma_kquant(hip, torch_gpu, oracle, qtype, m, n, k):
    torch = torch_gpu
    say(f"mfma type={qtype} {m}x{n}x{k}")
    act, w = oracle.create_input(qtype, m, n, k, seed=m * 13 + n + qtype)
    aq = oracle.quantize_q8_K(act)
    got = run_mul_mat(hip, torch, qtype, w, aq, m, n, k, hip.PATH_MFMA)
    check_close(oracle, qtype, got, w, aq, m, n, k, label=f"mfma type={qtype} {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(470, 1500, 1536), (300, 2000, 1024), (480, 1536, 1536)])
def test_mfma_q4_K_whole_k_tiles(hip, torch_gpu, oracle, m, n, k):
    """Shapes the whole-K q4_K tiles take (k = 1024 or 1536, half to one 32 x 96
    tile per CU), ragged edges included, against the oracle's bound."""
    torch = torch_gpu
    say(f"q4_K whole-K tiles {m}x{n}x{k}")
    act, w = oracle.create_input(1, m, n, k, seed=m + n)
    aq = oracle.quantize_q8_K(act)
    got = run_mul_mat(hip, torch, 1, w, aq, m, n, k, hip.PATH_MFMA)
    check_close(oracle, 1, got, w, aq, m, n, k, label=f"q4_K whole-K {m}x{n}x{k}")


def test_config2_q4_K_full_size(hip, torch_gpu, oracle):
    """c2: q4_K x q8_K M=480 N=1536 K=1536 through pfng_hip_compute, whole output
    checked; then weight-row permutation equivariance and exact doubling with
    the weight scales on the product."""
    torch = torch_gpu
    m, n, k = 480, 1536, 1536
    say("c2 q4_K 480x1536x1536")
    act, w = oracle.create_input(1, m, n, k, seed=1)
    wt, at = dev(torch, w), dev(torch, act)
    got = hip.compute(1, at, wt, n)
    torch.cuda.synchronize()
    aq = oracle.quantize_q8_K(act)
    check_close(oracle, 1, got.cpu().numpy(), w, aq, m, n, k, label="c2")
    aq_t = hip.quantize_q8_K(at)
    prod = hip.mul_mat(1, wt, aq_t, m, n, k)
    torch.cuda.synchronize()
    assert torch.equal(prod, got)
    check_full_size_properties(hip, torch, 1, w, wt, aq_t, prod, m, n, k)


def test_config3_iq2_xxs_full_size_sampled(hip, torch_gpu, oracle):
    """c3: iq2_xxs x q8_K M=512 N=4096 K=4096 with the baseline weight generator;
    oracle on 48 seeded rows, activation-row and weight-row permutation
    equivariance, exact doubling with the weight scales."""
    torch = torch_gpu
    m, n, k = 512, 4096, 4096
    say("c3 iq2_xxs 512x4096x4096")
    act, w = oracle.create_input(2, m, n, k, seed=1, variant=1)
    wt, at = dev(torch, w), dev(torch, act)
    aq_t = hip.quantize_q8_K(at)
    got = hip.mul_mat(2, wt, aq_t, m, n, k)
    torch.cuda.synchronize()
    aq = oracle.quantize_q8_K(act)
    assert np.array_equal(aq_t.cpu().numpy().reshape(-1), aq.view(np.uint8).reshape(-1))
    g = got.cpu().numpy()
    assert np.isfinite(g).all()
    rows = np.sort(np.random.default_rng(6).choice(m, 48, replace=False))
    check_close(oracle, 2, g, w, aq, m, n, k, rows=rows, label="c3")
    perm = torch.randperm(m, generator=torch.Generator().manual_seed(0)).cuda()
    got_p = hip.mul_mat(2, wt, aq_t[perm].contiguous(), m, n, k)
    torch.cuda.synchronize()
    assert torch.equal(got_p, got[perm])
    check_full_size_properties(hip, torch, 2, w, wt, aq_t, got, m, n, k)


# ------------------------------------------------- small-shape configs ----

@pytest.mark.parametrize("qtype,m,n,k", [(0, 480, 1536, 1536), (0, 9, 300, 640), (0, 200, 130, 1024),
                                         (0, 33, 65, 256), (0, 16, 4096, 4096), (0, 40, 200, 2048),
                                         (1, 480, 1536, 1536), (1, 100, 77, 512), (1, 16, 4096, 4096),
                                         (1, 32, 11008, 2048), (2, 130, 200, 2048), (2, 31, 33, 256),
                                         (2, 9, 300, 1024), (2, 480, 1536, 1536), (2, 64, 4096, 4096)])
def test_small_shapes_deterministic_and_correct(hip, torch_gpu, oracle, qtype, m, n, k):
    """Shapes that take the 32x32-tile configurations (two or, for q4_0 decode
    batches, eight waves share each stage's blocks; for the K-quants, 2 or 4
    slices take alternate super-blocks, idle ones included when nb < 4; all add
    their partials through LDS): within tolerance, and bit-identical across
    repeated launches and after a launch of another shape."""
    torch = torch_gpu
    say(f"small shape type={qtype} {m}x{n}x{k}")
    act, w = oracle.create_input(qtype, m, n, k, seed=m + n + k + qtype)
    aq = oracle.quantize_activation(qtype, act)
    wt, at = dev(torch, w), dev(torch, aq)
    first = hip.mul_mat(qtype, wt, at, m, n, k, path=hip.PATH_MFMA)
    torch.cuda.synchronize()
    check_close(oracle, qtype, first.cpu().numpy(), w, aq, m, n, k, label=f"small type={qtype} {m}x{n}x{k}")
    for _ in range(3):
        again = hip.mul_mat(qtype, wt, at, m, n, k, path=hip.PATH_MFMA)
    act2, w2 = oracle.create_input(qtype, 64, 96, k, seed=3)
    hip.mul_mat(qtype, dev(torch, w2), dev(torch, oracle.quantize_activation(qtype, act2)), 64, 96, k,
                path=hip.PATH_MFMA)
    last = hip.mul_mat(qtype, wt, at, m, n, k, path=hip.PATH_MFMA)
    torch.cuda.synchronize()
    assert torch.equal(first, again) and torch.equal(first, last)


def test_mfma_in_graph_replays(hip, torch_gpu, oracle):
    """c0 captured into a graph: every replay equals the eager result."""
    torch = torch_gpu
    m, n, k = 480, 1536, 1536
    say("graph replay c0")
    act, w = oracle.create_input(0, m, n, k, seed=1)
    wt, at = dev(torch, w), dev(torch, oracle.quantize_q8_0(act))
    s = torch.cuda.Stream()
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    with torch.cuda.stream(s):
        hip.mul_mat(0, wt, at, m, n, k, out=out)
    s.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        hip.mul_mat(0, wt, at, m, n, k, out=out)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


# ------------------------------------------------------- q4_K / iq2_xxs GEMV ----

@pytest.mark.parametrize("qtype", [1, 2])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 13, 16])
@pytest.mark.parametrize("n,k", [(4096, 4096), (257, 1536), (64, 256), (33, 8192), (20, 20480), (8, 65536),
                                 (37, 4096)])
def test_gemv_kquant(hip, torch_gpu, oracle, qtype, m, n, k):
    """m = 1: q4_K copies the activation row into LDS while it fits 64 KB
    (k <= 57344; k = 65536 takes the global-read kernel), iq2_xxs reads it from
    global memory; m = 2..16 stage the rows in LDS while m * (k / 256) * 320 +
    3072 bytes fit 160 KB (at k = 20480 only m <= 6 do, at k = 65536 none; the
    others up to m = 8 take the global-read kernel). At q4_K k % 1024 == 0 and
    iq2_xxs k % 2048 == 0 the one-chunk MFMA tile kernel takes q4_K from m = 5
    (k >= 4096) and iq2_xxs from m = 9 at k = 4096 (m = 5..8 there: the
    two-half-copy tile) and from m = 5 above, one super-block per wave and
    round (16 rounds at k = 65536)."""
    tiles = k % (1024 if qtype == 1 else 2048) == 0
    if m > 8 and not tiles and m * (k // 256) * 320 + 3072 > 160 * 1024:
        pytest.skip("m > 8 takes the GEMV below the tiles' k only while the staged activations fit in LDS")
    torch = torch_gpu
    say(f"gemv type={qtype} m={m} n={n} k={k}")
    act, w = oracle.create_input(qtype, m, n, k, seed=m * 31 + n + qtype)
    aq = oracle.quantize_q8_K(act)
    got = run_mul_mat(hip, torch, qtype, w, aq, m, n, k, hip.PATH_GEMV)
    check_close(oracle, qtype, got, w, aq, m, n, k, label=f"gemv type={qtype} m={m} n={n} k={k}")


@pytest.mark.parametrize("qtype", [1, 2])
def test_gemv_kquant_random_bytes_and_extremes(hip, torch_gpu, oracle, qtype):
    torch = torch_gpu
    m, n, k = 4, 130, 2304
    say(f"gemv random bytes type={qtype}")
    w = random_weight_blocks(oracle, qtype, n, k, seed=41 + qtype)
    for aq in (oracle.quantize_q8_K(oracle.create_input(qtype, m, 1, k, seed=2)[0]),
               extreme_activation(oracle, m, k, seed=5)):
        got = run_mul_mat(hip, torch, qtype, w, aq, m, n, k, hip.PATH_GEMV)
        check_close(oracle, qtype, got, w, aq, m, n, k, label=f"gemv random bytes type={qtype}")
        # the automatic path takes the GEMV for m <= 8
        auto = run_mul_mat(hip, torch, qtype, w, aq, m, n, k, hip.PATH_AUTO)
        assert np.array_equal(auto, got)


@pytest.mark.parametrize("qtype", [1, 2])
@pytest.mark.parametrize("m", list(range(5, 17)) + [17, 20, 31, 32, 33, 47, 48, 49, 63, 64, 65, 96, 127, 128])
@pytest.mark.parametrize("n", [4096, 37, 1])
def test_gemv_kquant_one_superblock_per_wave(hip, torch_gpu, oracle, qtype, m, n):
    """k = 4096, m = 5..128: 16-row MFMA tiles with one super-block per wave
    (from m = 17 over chunks of 16 activation rows, each chunk's halves
    refilled while the other half is multiplied),
    each wave's weight and activation blocks copied in two halves of 16-byte
    chunks from the 16-byte boundary before them (a different offset for each
    wave). Every m, a partial last tile and a single weight row; the
    generator's inputs, then random weight bytes (every scale, min, grid index
    and sign pattern) against extreme activations."""
    torch = torch_gpu
    k = 4096
    say(f"gemv one super-block per wave type={qtype} m={m} n={n}")
    act, w = oracle.create_input(qtype, m, n, k, seed=m * 7 + n + qtype)
    aq = oracle.quantize_q8_K(act)
    got = run_mul_mat(hip, torch, qtype, w, aq, m, n, k, hip.PATH_GEMV)
    check_close(oracle, qtype, got, w, aq, m, n, k, label=f"gemv sb type={qtype} m={m} n={n}")
    wr = random_weight_blocks(oracle, qtype, n, k, seed=59 + m + qtype)
    ax = extreme_activation(oracle, m, k, seed=m)
    got = run_mul_mat(hip, torch, qtype, wr, ax, m, n, k, hip.PATH_GEMV)
    check_close(oracle, qtype, got, wr, ax, m, n, k, label=f"gemv sb random bytes type={qtype} m={m} n={n}")


@pytest.mark.parametrize("m", [5, 6, 9, 16, 17, 33, 64, 128])
@pytest.mark.parametrize("qtype,n,k", [(0, 512, 8192), (0, 37, 12288), (0, 256, 14336), (0, 37, 11008), (0, 64, 4352),
                                       (1, 512, 8192), (1, 37, 12288), (1, 256, 14336), (1, 37, 5120),
                                       (2, 512, 8192), (2, 37, 12288), (2, 256, 14336), (2, 37, 6144)])
def test_gemv_tiles_several_rounds(hip, torch_gpu, oracle, qtype, m, n, k):
    """Above k = 4096: the one-chunk (m <= 16) and chunked MFMA tile GEMVs give
    wave w the K groups w, w + 16, ... (q4_0: 8 blocks, K-quants: one
    super-block), one per round, the partial sums carried across rounds in
    registers; at k = 4352, 5120, 6144, 11008 and 14336 the waves run different
    numbers of rounds (k = 4352: wave 0 two, the others one). From m = 5 the
    automatic path takes the GEMV for every case; the generator's inputs, then
    random weight bytes against activations at the int8 limits, 37 columns a
    partial tile."""
    torch = torch_gpu
    say(f"gemv rounds type={qtype} m={m} n={n} k={k}")
    assert hip.auto_path(qtype, m, n, k) == hip.PATH_GEMV
    quantize = oracle.quantize_q8_0 if qtype == 0 else oracle.quantize_q8_K
    act, w = oracle.create_input(qtype, m, n, k, seed=m * 17 + n + qtype)
    aq = quantize(act)
    got = run_mul_mat(hip, torch, qtype, w, aq, m, n, k, hip.PATH_AUTO)
    check_close(oracle, qtype, got, w, aq, m, n, k, label=f"gemv rounds type={qtype} m={m} n={n} k={k}")
    wr = random_weight_blocks(oracle, qtype, n, k, seed=83 + m + qtype)
    ax = quantize(np.where(np.random.default_rng(m + qtype).random((m, k)) < 0.5, -1.0, 1.0).astype(np.float32))
    got = run_mul_mat(hip, torch, qtype, wr, ax, m, n, k, hip.PATH_AUTO)
    check_close(oracle, qtype, got, wr, ax, m, n, k, label=f"gemv rounds random bytes type={qtype} m={m} n={n} k={k}")


# ------------------------------------------------------ weight quantizers ----

def weight_test_matrix(rows, k, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, k)) * rng.uniform(1e-4, 30, (rows, 1))).astype(np.float32)
    x[0] = 0.0                                   # all-zero blocks (d = -0.0 for q4_0)
    x[1, :64] = 7.0                              # constant blocks / sub-blocks
    x[2, :256] = np.linspace(-1, 1, 256)         # ties at the rounding points
    x[3, ::2] = -x[3, 1::2]                      # equal magnitudes of both signs (first one wins)
    x[4, :256] = np.abs(x[4, :256]) + 1.0        # all positive: negative mins
    x[5, :256] = -np.abs(x[5, :256]) - 1.0       # all negative
    x[6, 32:64] = np.float32(3.0) + np.float32(1e-6) * np.arange(32, dtype=np.float32)  # tiny range
    return x


@pytest.mark.parametrize("qtype", [0, 1])
@pytest.mark.parametrize("rows,k", [(37, 1024), (1, 256), (300, 4096)])
def test_weight_quantizer_bit_exact(hip, torch_gpu, oracle, qtype, rows, k):
    torch = torch_gpu
    say(f"weight quantizer type={qtype} rows={rows} k={k}")
    x = weight_test_matrix(max(rows, 8), k, seed=qtype + k)[:rows] if rows >= 8 else \
        np.random.default_rng(1).uniform(-1, 1, (rows, k)).astype(np.float32)
    got = hip.quantize_weights_gpu(qtype, dev(torch, x))
    torch.cuda.synchronize()
    expect = oracle.quantize_q4_0(x) if qtype == 0 else oracle.quantize_q4_K(x)
    assert np.array_equal(got.cpu().numpy().reshape(-1), expect.view(np.uint8).reshape(-1))


def test_weight_quantizer_matches_reference_generator(hip, torch_gpu, oracle):
    """The device quantizers reproduce the reference harness's weights for
    seed 1 (draws from the product's host generator, quantized on the GPU)."""
    torch = torch_gpu
    say("weight quantizer vs create_input")
    for qtype, (m, n, k) in ((0, (2, 64, 1536)), (1, (2, 64, 1536))):
        import numpy as _np
        rng_act, w_ref = oracle.create_input(qtype, m, n, k, seed=1, variant=0)
        # the weights' fp32 draws follow the activations' in the same mt19937 stream
        draws = oracle.uniform_real_draws(1, -1.0, 1.0, m * k + n * k)[m * k:].reshape(n, k)
        got = hip.quantize_weights_gpu(qtype, dev(torch, _np.ascontiguousarray(draws, dtype=_np.float32)))
        torch.cuda.synchronize()
        assert _np.array_equal(got.cpu().numpy().reshape(-1), _np.ascontiguousarray(w_ref).view(_np.uint8).reshape(-1))


# ------------------------------------------------ fused quantize + GEMV ----

@pytest.mark.parametrize("m", [1, 2, 5, 7, 8, 12, 16])
@pytest.mark.parametrize("n,k", [(4096, 4096), (300, 64), (129, 7680), (64, 1536)])
def test_compute_fused_gemv(hip, torch_gpu, oracle, m, n, k):
    """pfng_hip_compute with q4_0: m <= 2 quantizes inside the GEMV kernel, larger
    m quantize first. The output matches the oracle's compute (quantize +
    product) within the bound and equals the separate quantize + GEMV result
    exactly (same q8_0 bytes; the fused kernel adds in the GEMVs' order)."""
    torch = torch_gpu
    if m <= 2 and (k // 32) * 34 * m > 65536:
        pytest.skip("activations exceed the fused kernel's LDS budget (covered by the unfused path)")
    say(f"fused gemv m={m} n={n} k={k}")
    act, w = oracle.create_input(0, m, n, k, seed=m + n + k)
    wt, at = dev(torch, w), dev(torch, act)
    fused = hip.compute(0, at, wt, n)
    torch.cuda.synchronize()
    aq = oracle.quantize_q8_0(act)
    check_close(oracle, 0, fused.cpu().numpy(), w, aq, m, n, k, label=f"fused m={m} n={n} k={k}")
    unfused = hip.mul_mat(0, wt, hip.quantize_q8_0(at), m, n, k, path=hip.PATH_GEMV)
    torch.cuda.synchronize()
    assert torch.equal(fused, unfused)


# q4_K / iq2_xxs at m == 1 quantize the q8_K row inside the GEMV's workgroups
# while it (with iq2_xxs's tables) fits 64 KB of LDS: k up to 56064 for q4_K
# (224 blocks), 53760 for iq2_xxs (210 blocks); longer rows quantize first.
@pytest.mark.parametrize("qtype", [1, 2])
@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (1, 300, 256), (1, 129, 7680), (1, 77, 53760), (1, 50, 57344),
                                   (2, 64, 1536)])
def test_compute_fused_kquant_gemv(hip, torch_gpu, oracle, qtype, m, n, k):
    """pfng_hip_compute with q4_K / iq2_xxs: within the bound of the oracle's
    compute, and equal to the separate quantize_q8_K + GEMV result bit for bit
    (same q8_K bytes, sums in the same order)."""
    torch = torch_gpu
    say(f"fused kquant gemv type={qtype} m={m} n={n} k={k}")
    act, w = oracle.create_input(qtype, m, n, k, seed=m + n + k)
    wt, at = dev(torch, w), dev(torch, act)
    fused = hip.compute(qtype, at, wt, n)
    torch.cuda.synchronize()
    aq = oracle.quantize_q8_K(act)
    check_close(oracle, qtype, fused.cpu().numpy(), w, aq, m, n, k, label=f"fused type={qtype} m={m} n={n} k={k}")
    unfused = hip.mul_mat(qtype, wt, hip.quantize_q8_K(at), m, n, k, path=hip.PATH_GEMV)
    torch.cuda.synchronize()
    assert torch.equal(fused, unfused)


@pytest.mark.parametrize("m", [3, 4, 5, 9, 16, 17, 64, 65, 128])
@pytest.mark.parametrize("qtype,n,k", [(0, 96, 512), (0, 37, 1024), (0, 64, 1536), (0, 50, 2048), (0, 40, 3072),
                                       (1, 96, 1024), (1, 37, 2048), (1, 50, 3072), (2, 64, 2048), (2, 37, 2048)])
def test_gemv_tiles_small_k(hip, torch_gpu, oracle, qtype, m, n, k):
    """Below k = 4096 the one-chunk and chunked MFMA tile GEMVs run with the
    waves past the last K group idle (q4_0 at k = 512: 14 of 16), from the m
    measured fastest for the format and k, up to m = 64 below k = 2048 and 128
    from there; the other m take the staged or pair kernels or the GEMM. An idle
    wave stores its zero partials in its own LDS region, where the iq2_xxs
    kernel's table copy also lands, so it waits for that copy first (without the
    wait iq2_xxs at k = 2048, m = 64 read table bytes as partials). The automatic path against the
    oracle, on the generator's inputs and on random weight bytes against
    activations at the int8 limits."""
    torch = torch_gpu
    say(f"gemv small k type={qtype} m={m} n={n} k={k}")
    if 9 <= m <= (128 if k >= 2048 else 64):
        assert hip.auto_path(qtype, m, n, k) == hip.PATH_GEMV
    quantize = oracle.quantize_q8_0 if qtype == 0 else oracle.quantize_q8_K
    act, w = oracle.create_input(qtype, m, n, k, seed=m * 5 + n + qtype)
    aq = quantize(act)
    got = run_mul_mat(hip, torch, qtype, w, aq, m, n, k, hip.PATH_AUTO)
    check_close(oracle, qtype, got, w, aq, m, n, k, label=f"gemv small k type={qtype} m={m} n={n} k={k}")
    wr = random_weight_blocks(oracle, qtype, n, k, seed=97 + m + qtype)
    ax = quantize(np.where(np.random.default_rng(m + 7).random((m, k)) < 0.5, -1.0, 1.0).astype(np.float32))
    got = run_mul_mat(hip, torch, qtype, wr, ax, m, n, k, hip.PATH_AUTO)
    check_close(oracle, qtype, got, wr, ax, m, n, k, label=f"gemv small k random bytes type={qtype} m={m} k={k}")


@pytest.mark.parametrize("qtype,m,n,k", [(0, 24, 96, 14336), (0, 7, 64, 11008), (1, 40, 64, 14336), (1, 9, 50, 5120),
                                         (2, 12, 80, 14336), (2, 70, 40, 8192)])
def test_compute_tiles_several_rounds(hip, torch_gpu, oracle, qtype, m, n, k):
    """pfng_hip_compute where the product is an MFMA tile GEMV over several
    rounds (quantize first, m >= 3): within the bound of the oracle's compute,
    and equal bit for bit to quantize + the GEMV called directly."""
    torch = torch_gpu
    say(f"compute rounds type={qtype} m={m} n={n} k={k}")
    assert hip.auto_path(qtype, m, n, k) == hip.PATH_GEMV
    act, w = oracle.create_input(qtype, m, n, k, seed=m * 3 + n + k)
    wt, at = dev(torch, w), dev(torch, act)
    got = hip.compute(qtype, at, wt, n)
    quantize = hip.quantize_q8_0 if qtype == 0 else hip.quantize_q8_K
    direct = hip.mul_mat(qtype, wt, quantize(at), m, n, k, path=hip.PATH_GEMV)
    torch.cuda.synchronize()
    aq = oracle.quantize_activation(qtype, act)
    check_close(oracle, qtype, got.cpu().numpy(), w, aq, m, n, k, label=f"compute rounds type={qtype} m={m} k={k}")
    assert torch.equal(got, direct)


def test_wrappers_reject_short_or_strided_buffers(hip, torch_gpu):
    """The C-ABI takes bare pointers; the Python wrappers check sizes, layout
    and device first and raise before anything is launched."""
    torch = torch_gpu
    say("wrapper argument checks")
    m, n, k = 4, 64, 256
    w = torch.zeros((n, (k // 32) * 18), dtype=torch.uint8, device="cuda")
    a = torch.zeros((m, (k // 32) * 34), dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError, match="weight holds"):
        hip.mul_mat(0, w[: n - 1], a, m, n, k)
    with pytest.raises(ValueError, match="act_q holds"):
        hip.mul_mat(0, w, a[: m - 1], m, n, k)
    with pytest.raises(ValueError, match="out holds"):
        hip.mul_mat(0, w, a, m, n, k, out=torch.empty((m, n - 1), dtype=torch.float32, device="cuda"))
    with pytest.raises(ValueError, match="contiguous"):
        hip.mul_mat(0, torch.zeros((n, 2 * (k // 32) * 18), dtype=torch.uint8, device="cuda")[:, ::2], a, m, n, k)
    with pytest.raises(ValueError, match="device tensor"):
        hip.quantize_q8_0(torch.zeros((m, k), dtype=torch.float32))
    x = torch.zeros((m, k), dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError, match="workspace holds"):
        hip.compute(0, x, w, n, workspace=torch.empty(8, dtype=torch.uint8, device="cuda"))
    torch.cuda.synchronize()
