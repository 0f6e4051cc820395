"""Pins the CPU oracle (oracle/pfng_oracle.c) — CPU only.

Each check is chosen so that a plausible restatement mistake fails it:
  * golden vectors produced by the reference's own code (tests/golden/, oracle/_ref);
  * the C++ standard's mt19937 known answer and an independent MT19937 (numpy);
  * fp16 conversions exhaustively against numpy's float16 (an independent IEEE implementation);
  * quantizer closed forms and invariants (|q| <= 127, amax -> +-127, bsums = sum q);
  * integer block sums against brute-force int64 numpy dots;
  * fp32 outputs against a float64 evaluation within the 1e-5 * sum|terms| contract.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_vectors():
    return np.load(os.path.join(GOLDEN, "ref_vectors.npz"))


CASES = [(0, 24, 32, 256), (0, 3, 5, 96), (1, 8, 16, 512), (2, 8, 16, 512)]


# ---------------------------------------------------------------- RNG ----

def test_mt19937_standard_known_answer(oracle):
    # [rand.predef]: the 10000th consecutive invocation of a default-constructed
    # std::mt19937 (seed 5489) produces 4123659995.
    assert int(oracle.mt_draws(5489, 10000)[-1]) == 4123659995


def test_mt19937_matches_numpy_legacy_seeding(oracle):
    # numpy's RandomState seeds MT19937 with init_genrand(seed) for integer seeds,
    # the same routine as std::mt19937(seed); it is an independent implementation.
    rs = np.random.RandomState(1)
    ref = rs.randint(0, 2**32, size=2000, dtype=np.uint64).astype(np.uint32)
    bg = np.random.MT19937()
    bg._legacy_seeding(1)
    raw = np.array([bg.random_raw() for _ in range(2000)], dtype=np.uint64).astype(np.uint32)
    ours = oracle.mt_draws(1, 2000)
    assert np.array_equal(ours, raw)
    assert ref.shape == ours.shape


def test_uniform_real_is_u_over_2_32(oracle):
    # generate_canonical<float, 24> over a 32-bit engine: one draw, u / 2^32 in float.
    u = oracle.mt_draws(1, 4096).astype(np.float64)
    expect = ((u.astype(np.float32) / np.float32(2.0**32)).astype(np.float32) * np.float32(2.0)).astype(np.float32)
    expect = (expect + np.float32(-1.0)).astype(np.float32)
    got = oracle.uniform_real_draws(1, -1.0, 1.0, 4096)
    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))
    assert got.min() >= -1.0 and got.max() < 1.0


# ---------------------------------------------------------------- fp16 ----

def test_fp16_to_fp32_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = oracle.fp16_to_fp32(h)
    ref = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(ours[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isinf(ours[np.isinf(ref)]))
    assert np.all(np.isnan(ours[np.isnan(ref)]))


def test_fp32_to_fp16_round_to_nearest_even(oracle):
    rng = np.random.default_rng(3)
    x = np.concatenate([
        rng.uniform(-70000, 70000, 200000).astype(np.float32),
        (rng.standard_normal(200000) * 1e-5).astype(np.float32),                    # fp16 subnormal range
        np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32),  # exact halves
        (np.arange(1, 65536, dtype=np.float32) + np.float32(0.5)),                   # ties in the integer range
    ])
    x = x[np.isfinite(x)]
    ours = oracle.fp32_to_fp16(x)
    ref = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x.astype(np.float16))
    assert np.array_equal(ours[~nan], ref[~nan])


def test_fp16_special_values_match_reference(oracle):
    e = np.load(os.path.join(GOLDEN, "ref_quant_edges.npz"))
    assert np.array_equal(oracle.fp32_to_fp16(e["fp16/x"]), e["fp16/y"])


# ---------------------------------------------------------- quantizers ----

@pytest.mark.parametrize("name", ["q8_0", "q8_K", "q4_0", "q4_K"])
def test_quantizer_edge_cases_match_reference_bytes(oracle, name):
    e = np.load(os.path.join(GOLDEN, "ref_quant_edges.npz"))
    x, y = e[f"{name}/x"], e[f"{name}/y"]
    fn = {"q8_0": oracle.quantize_q8_0, "q8_K": oracle.quantize_q8_K,
          "q4_0": oracle.quantize_q4_0, "q4_K": oracle.quantize_q4_K}[name]
    got = fn(x).view(np.uint8).reshape(y.shape)
    assert np.array_equal(got, y)


def _q8_closed_form(x, qk):
    """numpy float32 statement of d = amax/127, q = round-half-away(x * (1/d))."""
    xb = x.reshape(-1, qk)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, (np.float32(1.0) / d).astype(np.float32), np.float32(0.0)).astype(np.float32)
    p = (xb * inv[:, None]).astype(np.float32)
    q = (np.sign(p) * np.floor(np.abs(p) + np.float32(0.5))).astype(np.int32)
    return d, q


def test_q8_0_closed_form_and_invariants(oracle):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((64, 512)) * rng.uniform(0.01, 100, (64, 1))).astype(np.float32)
    y = oracle.quantize_q8_0(x).reshape(-1)
    d, q = _q8_closed_form(x, 32)
    assert np.array_equal(y["qs"].astype(np.int32), q)
    assert np.array_equal(y["d"], d.astype(np.float16).view(np.uint16))
    assert np.abs(y["qs"].astype(int)).max() <= 127
    # the element at |x| = amax maps to +-127
    xb = x.reshape(-1, 32)
    i = np.abs(xb).argmax(axis=1)
    assert np.all(np.abs(y["qs"][np.arange(len(i)), i].astype(int)) == 127)


def test_q8_K_closed_form_bsums(oracle):
    rng = np.random.default_rng(12)
    x = (rng.standard_normal((16, 1024)) * 3).astype(np.float32)
    y = oracle.quantize_q8_K(x).reshape(-1)
    d, q = _q8_closed_form(x, 256)
    assert np.array_equal(y["qs"].astype(np.int32), q)
    assert np.array_equal(y["d"].view(np.uint32), d.view(np.uint32))
    assert np.array_equal(y["bsums"].astype(np.int32), q.reshape(-1, 16, 16).sum(axis=2))


def test_q4_0_quantizer_reconstruction(oracle):
    # value = (nib - 8) * d with d = signed_max / -8: the signed maximum maps to nibble 0
    rng = np.random.default_rng(13)
    x = rng.uniform(-1, 1, (32, 256)).astype(np.float32)
    y = oracle.quantize_q4_0(x).reshape(-1)
    xb = x.reshape(-1, 32)
    lo = (y["qs"] & 15).astype(int)
    hi = (y["qs"] >> 4).astype(int)
    q = np.concatenate([lo, hi], axis=1)
    d = y["d"].view(np.float16).astype(np.float32)
    i = np.abs(xb).argmax(axis=1)
    assert np.all(q[np.arange(len(i)), i] == 0)
    err = np.abs((q - 8) * d[:, None] - xb)
    ad = np.abs(d)[:, None]
    # round-to-nearest (x*id + 8.5 truncated) within the nibble range; the top code
    # 15 also absorbs x*id in (6.5, 8], an error of up to one step
    assert np.all(err[q < 15] <= (0.5 * ad * 1.002 + 1e-7).repeat(32, axis=1)[q < 15])
    assert np.all(err <= ad * 1.002 + 1e-7)


# ------------------------------------------------------ reference vectors ----

@pytest.mark.parametrize("case", CASES, ids=lambda c: f"t{c[0]}_{c[1]}x{c[2]}x{c[3]}")
def test_generator_quantizer_compute_match_reference_vectors(oracle, case):
    t, m, n, k = case
    tag = f"{oracle.TYPE_NAMES[t]}_{m}x{n}x{k}"
    v = load_vectors()
    act, w = oracle.create_input(t, m, n, k, seed=1, variant=0)
    assert np.array_equal(act.view(np.uint32), v[f"{tag}/act"].view(np.uint32))
    assert np.array_equal(w.view(np.uint8).reshape(-1), v[f"{tag}/weight"].reshape(-1))
    aq = oracle.quantize_activation(t, act)
    assert np.array_equal(aq.view(np.uint8).reshape(-1), v[f"{tag}/act_q"].reshape(-1))
    out = oracle.compute(t, act, w, threads=1)
    assert np.array_equal(out.view(np.uint32), v[f"{tag}/out"].view(np.uint32))


def test_documented_preflight_checksum(oracle):
    # kernels/q4_0-q8_0-IME-m4i/implementations/smt-ime1/performance.md:63-65: a
    # q4_0 kernel at M=24 N=32 K=256 (seed 1) verified with max_abs 1.90735e-06
    # against the oracle and printed checksum 3.84864689. The oracle's own
    # checksum must sit within that verification distance.
    act, w = oracle.create_input(0, 24, 32, 256, seed=1, variant=0)
    out = oracle.compute(0, act, w, threads=1)
    cs = oracle.checksum(out)
    assert abs(cs - 3.84864689) <= 3 * 1.90735e-06
    assert abs(cs - 3.8486468121409416) < 1e-12


@pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(GOLDEN), "..", "oracle", "_ref", "libpfng_ref.so")),
                    reason="oracle/_ref not built (reference tree absent)")
@pytest.mark.parametrize("t,m,n,k", [(0, 7, 9, 512), (1, 5, 7, 768), (2, 5, 7, 768)])
def test_oracle_matches_reference_build_other_shapes(oracle, t, m, n, k):
    R = oracle.ref()
    act, w = oracle.create_input(t, m, n, k, seed=5, variant=0)
    ra = np.empty_like(act)
    rw = np.zeros_like(w)
    assert R.ref_create_input(t, 5, m, n, k, oracle._ptr(ra), oracle._ptr(rw)) == 0
    assert np.array_equal(act.view(np.uint32), ra.view(np.uint32)) and w.tobytes() == rw.tobytes()
    out = oracle.compute(t, act, w, threads=2)
    rout = np.zeros_like(out)
    assert R.ref_compute(t, oracle._ptr(act), oracle._ptr(w), oracle._ptr(rout), m, n, k) == 0
    assert np.array_equal(out.view(np.uint32), rout.view(np.uint32))


@pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(GOLDEN), "..", "oracle", "_ref", "libpfng_ref.so")),
                    reason="oracle/_ref not built (reference tree absent)")
@pytest.mark.parametrize("t,m,n,k,threads", [(0, 1, 37, 512, 4), (0, 6, 9, 256, 16), (1, 3, 11, 512, 3),
                                             (2, 2, 13, 512, 5)])
def test_threaded_reference_compute_equals_reference_compute(oracle, t, m, n, k, threads):
    """The all-core CPU baseline splits llama_reference::compute's output columns
    over threads; every element must stay bit-identical."""
    R = oracle.ref()
    act, w = oracle.create_input(t, m, n, k, seed=9, variant=0)
    a = np.zeros((m, n), np.float32)
    b = np.zeros((m, n), np.float32)
    assert R.ref_compute(t, oracle._ptr(act), oracle._ptr(w), oracle._ptr(a), m, n, k) == 0
    assert R.ref_compute_threads(t, oracle._ptr(act), oracle._ptr(w), oracle._ptr(b), m, n, k, threads) == 0
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---------------------------------------------------------- iq2 tables ----

def test_iq2xxs_grid_and_signs_match_reference_tables(oracle):
    import ctypes
    tab = json.load(open(os.path.join(GOLDEN, "iq2xxs_tables.json")))
    grid = [int(v, 16) for v in tab["iq2xxs_grid"]]
    # decode every grid entry through the oracle's sub-block decoder: a sub-block
    # whose four groups all use entry e with zero signs yields grid bytes of e
    for e in range(256):
        packed = np.array([e, e, e, e, 0, 0, 0, 0], np.uint8)
        vals = np.zeros(32, np.int8)
        sc = ctypes.c_int(0)
        oracle.lib().pfo_iq2_xxs_decode_subblock(oracle._ptr(packed), oracle._ptr(vals), ctypes.byref(sc))
        expect = np.frombuffer(np.uint64(grid[e]).tobytes(), np.uint8).astype(np.int8)
        assert np.array_equal(vals[:8], expect)
        assert sc.value == 1
    # the reference generator's 32-entry grid is a prefix of the full grid
    assert [int(v, 16) for v in tab["reduced_grid_32"]] == grid[:32]
    # sign table entry i == i | parity(i) << 7
    for i, s in enumerate(tab["ksigns_iq2xs"]):
        assert s == i | ((bin(i).count("1") & 1) << 7)
    # signs and scale: set sign index 0b0000011 (parity 0) on group 0 and scale 5
    packed = np.array([0, 0, 0, 0, 0, 0, 0, 0], np.uint8)
    sas = 0b0000011 | (5 << 28)
    packed[4:8] = np.frombuffer(np.uint32(sas).tobytes(), np.uint8)
    vals = np.zeros(32, np.int8)
    sc = ctypes.c_int(0)
    oracle.lib().pfo_iq2_xxs_decode_subblock(oracle._ptr(packed), oracle._ptr(vals), ctypes.byref(sc))
    assert list(vals[:8]) == [-8, -8, 8, 8, 8, 8, 8, 8] and sc.value == 11


# ------------------------------------------------------- integer sums ----

def _decode_q4_0(w):
    lo = (w["qs"] & 15).astype(np.int64) - 8
    hi = (w["qs"] >> 4).astype(np.int64) - 8
    return np.concatenate([lo, hi], axis=-1)  # (..., 32) in element order


def test_q4_0_isums_brute_force(oracle):
    act, w = oracle.create_input(0, 5, 7, 320, seed=3)
    aq = oracle.quantize_q8_0(act)
    got = oracle.isums(0, w, aq, 5, 7, 320)
    wv = _decode_q4_0(w)                     # (7, 10, 32)
    av = aq["qs"].astype(np.int64)           # (5, 10, 32)
    expect = np.einsum("nbe,mbe->mnb", wv, av)
    assert np.array_equal(got, expect)


def test_q4_K_isums_brute_force(oracle):
    m, n, k = 3, 4, 512
    act, w = oracle.create_input(1, m, n, k, seed=4)
    aq = oracle.quantize_q8_K(act)
    got = oracle.isums(1, w, aq, m, n, k)
    sc = np.zeros(w.shape + (8,), np.int64)
    mn = np.zeros(w.shape + (8,), np.int64)
    s = w["scales"].astype(np.int64)
    for i in range(4):  # llama_reference.cpp:116-121
        sc[..., i] = s[..., i] & 63
        sc[..., i + 4] = (s[..., i + 8] & 15) | ((s[..., i] >> 6) << 4)
        mn[..., i] = s[..., i + 4] & 63
        mn[..., i + 4] = (s[..., i + 8] >> 4) | ((s[..., i + 4] >> 6) << 4)
    q = np.zeros(w.shape + (256,), np.int64)
    for sb in range(8):
        packed = w["qs"][..., (sb // 2) * 32:(sb // 2) * 32 + 32].astype(np.int64)
        q[..., sb * 32:(sb + 1) * 32] = (packed & 15) if sb % 2 == 0 else (packed >> 4)
    a = aq["qs"].astype(np.int64)
    S = np.einsum("nbjs,mbjs->mnbj", q.reshape(n, -1, 8, 32), a.reshape(m, -1, 8, 32))
    isc = np.einsum("mnbj,nbj->mnb", S, sc)
    bs = aq["bsums"].astype(np.int64).reshape(m, -1, 8, 2).sum(axis=-1)
    imn = np.einsum("mbj,nbj->mnb", bs, mn)
    assert np.array_equal(got[..., 0], isc) and np.array_equal(got[..., 1], imn)
    # bsums pairing: bsum_2j + bsum_2j+1 equals the sum of sub-block j of q8_K
    assert np.array_equal(bs, a.reshape(m, -1, 8, 32).sum(axis=-1))


def test_iq2_isums_brute_force(oracle):
    m, n, k = 3, 4, 512
    act, w = oracle.create_input(2, m, n, k, seed=6, variant=1)
    aq = oracle.quantize_q8_K(act)
    got = oracle.isums(2, w, aq, m, n, k)
    tab = json.load(open(os.path.join(GOLDEN, "iq2xxs_tables.json")))
    grid = np.array([np.frombuffer(np.uint64(int(v, 16)).tobytes(), np.uint8) for v in tab["iq2xxs_grid"]], np.int64)
    packed = w["qs"].view(np.uint8).reshape(n, -1, 8, 8)  # (n, blocks, subblock, 8 bytes)
    sas = packed[..., 4:8].copy().view(np.uint32)[..., 0].astype(np.int64)
    vals = np.zeros((n, packed.shape[1], 8, 32), np.int64)
    for g in range(4):
        idx = (sas >> (7 * g)) & 0x7F
        par = np.array([bin(int(i)).count("1") & 1 for i in idx.reshape(-1)]).reshape(idx.shape)
        signs = idx | (par << 7)
        mags = grid[packed[..., g].astype(np.int64)]
        for l in range(8):
            neg = (signs >> l) & 1
            vals[..., g * 8 + l] = np.where(neg == 1, -mags[..., l], mags[..., l])
    scale = 2 * ((sas >> 28) & 15) + 1
    a = aq["qs"].astype(np.int64).reshape(m, -1, 8, 32)
    S = np.einsum("nbjs,mbjs->mnbj", vals, a)
    assert np.array_equal(got, np.einsum("mnbj,nbj->mnb", S, scale))
    assert grid[packed[..., :4].astype(np.int64)].max() == 43  # generator reaches the full grid


# ------------------------------------------------------- fp32 outputs ----

@pytest.mark.parametrize("t,m,n,k", [(0, 6, 10, 1024), (1, 4, 6, 1024), (2, 4, 6, 1024)])
def test_outputs_within_bound_of_float64(oracle, t, m, n, k):
    act, w = oracle.create_input(t, m, n, k, seed=9)
    aq = oracle.quantize_activation(t, act)
    out = oracle.matmul(t, w, aq, m, n, k, threads=1)
    terms = oracle.abs_terms(t, w, aq, m, n, k)
    isum = oracle.isums(t, w, aq, m, n, k)
    # float64 evaluation of the same quantized product
    if t == 0:
        dw = w["d"].view(np.float16).astype(np.float64)
        da = aq["d"].view(np.float16).astype(np.float64)
        exact = np.einsum("mnb,nb,mb->mn", isum.astype(np.float64), dw, da)
    elif t == 1:
        d = w["d"].view(np.float16).astype(np.float64)
        dmin = w["dmin"].view(np.float16).astype(np.float64)
        ad = aq["d"].astype(np.float64)
        exact = (np.einsum("mnb,nb,mb->mn", isum[..., 0].astype(np.float64), d, ad)
                 - np.einsum("mnb,nb,mb->mn", isum[..., 1].astype(np.float64), dmin, ad))
    else:
        d = w["d"].view(np.float16).astype(np.float64)
        ad = aq["d"].astype(np.float64)
        exact = 0.125 * np.einsum("mnb,nb,mb->mn", isum.astype(np.float64), d, ad)
    ok, worst, _ = oracle.within_tolerance(out, exact, terms)
    assert ok, worst
    # a dropped term would not pass: perturb one block's contribution
    assert not oracle.within_tolerance(out, exact + 0.01 * terms + 1e-3, terms)[0]
