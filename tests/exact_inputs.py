"""Inputs on which every fp32 step of the three products is exact.

Every scale is a power of two: the weights' fp16 ``d`` (and q4_K's ``dmin``),
q8_0's fp16 ``d`` and q8_K's fp32 ``d``. Their exponents are
``base_w + f(b) + g(n)`` for weight row n, block b and ``base_a - f(b) + h(m)``
for activation row m, with random f, g, h in {0, 1}: every scale varies by
block and by row, while the scale products of one output (m, n) share the
exponent ``g(n) + h(m)``. (q4_K's ``dmin`` is ``d`` or ``2 d`` at random.) The
int8 activation magnitudes are bounded so that, for every output, the sum
over all K elements of |term|, counted in units of the smallest power of two
that each of its terms is a multiple of, stays below 2**24. Terms per
element (llama_reference.cpp:113-161):

  q4_0    (q - 8) * a * dw * da
  q4_K    a * d * sc * q * ad  and  a * dmin * m * ad   (counted separately)
  iq2_xxs (2 s + 1) * v * a * 0.125 * d * ad

Any product of an integer with these scales, and any partial sum of any
subset of these terms, is then an integer multiple of that unit below 2**24
in magnitude, so it is exactly representable in fp32. Every summation order
and grouping gives the same bits. A correct kernel's output therefore equals
the oracle's (the reference's order) bit for bit. An integer block sum that
is off by one changes the output by a nonzero representable amount, so the
bitwise comparison fails.

Activations are built as fp32 rows x = q * 2**e. Each q8 block (q8_0: 32
values, q8_K: 256) holds one element at +-127, so quantize_row_q8_0/q8_K
(llama_reference.cpp:38-70) recover exactly d = 2**e and the integers q. The
same rows therefore drive the fused quantize + product kernels.
"""
from __future__ import annotations

import json
import os

import numpy as np

LIMIT = 2 ** 24
_GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_grid_bytes = None

# base exponents of the weight and activation scales, by weight type
_BASE_W = {0: -6, 1: -7, 2: -8}
_BASE_A = -7


def iq2_grid_bytes() -> np.ndarray:
    """256 x 8 magnitude bytes of the iq2_xxs grid (the fixture copied from the
    reference's ggml_min.h:69-134 table)."""
    global _grid_bytes
    if _grid_bytes is None:
        with open(os.path.join(_GOLDEN, "iq2xxs_tables.json")) as f:
            grid = [int(v, 16) for v in json.load(f)["iq2xxs_grid"]]
        _grid_bytes = np.array(grid, dtype="<u8").view(np.uint8).reshape(256, 8)
    return _grid_bytes


def _fp16_pow2(e: np.ndarray) -> np.ndarray:
    """fp16 bit patterns of 2**e (normal exponents only)."""
    assert ((e >= -14) & (e <= 15)).all()
    return ((e + 15).astype(np.uint16) << np.uint16(10)).astype(np.uint16)


def _pow2(e: np.ndarray) -> np.ndarray:
    return np.ldexp(1.0, np.asarray(e, dtype=np.int64))


def exact_weights(oracle, qtype: int, n: int, k: int, f: np.ndarray, g: np.ndarray, rng,
                  narrow: bool = False) -> np.ndarray:
    """Weight blocks with uniformly random payload bytes (every nibble, 6-bit
    scale and min, grid index, sign index and 4-bit scale) and fp16 scales
    2**(base + f[b] + g[n]). narrow: q4_K scales and mins <= 15, iq2_xxs
    scale nibbles <= 3 (for the longest rows)."""
    dt = oracle.WEIGHT_DTYPE[qtype]
    nb = k // oracle.QK[qtype]
    raw = rng.integers(0, 256, n * nb * dt.itemsize, dtype=np.uint8)
    w = raw.view(dt).reshape(n, nb).copy()
    e = _BASE_W[qtype] + f[None, :] + g[:, None]
    w["d"] = _fp16_pow2(e)
    if qtype == oracle.Q4_K:
        w["dmin"] = _fp16_pow2(e + rng.integers(0, 2, (n, nb)))
        if narrow:
            w["scales"][..., :8] &= 0x0F
    elif qtype == oracle.IQ2_XXS and narrow:
        b = np.ascontiguousarray(w["qs"]).view(np.uint8).reshape(n, nb, 8, 8)
        b[..., 7] &= 0x3F
        w["qs"] = b.reshape(n, nb, 64).view("<u2")
    return w


def exact_activation_rows(qtype: int, m: int, k: int, r: int, f: np.ndarray, h: np.ndarray, rng):
    """fp32 rows x = q * 2**e: |q| <= r except one +-127 per q8 block, e =
    base - f[b] + h[m]. Returns (x, q as int8 (m, k), e (m, blocks))."""
    qk = 32 if qtype == 0 else 256
    nb = k // qk
    q = rng.integers(-r, r + 1, (m, nb, qk)).astype(np.int8)
    pos = rng.integers(0, qk, (m, nb))
    sign = np.where(rng.random((m, nb)) < 0.5, -127, 127).astype(np.int8)
    np.put_along_axis(q, pos[..., None], sign[..., None], axis=2)
    e = _BASE_A - f[None, :] + h[:, None]
    x = (q.astype(np.float64) * _pow2(e)[..., None]).astype(np.float32).reshape(m, k)
    return x, q.reshape(m, k), e


def _weight_magnitudes(oracle, qtype: int, w: np.ndarray, k: int) -> np.ndarray:
    """Per weight element the factor of |term| that multiplies |a| * ad, as a
    float64 (n, k) array (q4_K: the d and dmin parts summed)."""
    n = w.shape[0]
    if qtype == oracle.Q4_0:
        qs = w["qs"].astype(np.int64)                       # (n, nb, 16)
        vals = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=2)
        dw = oracle.fp16_to_fp32(w["d"]).astype(np.float64)
        return (np.abs(vals) * dw[..., None]).reshape(n, k)
    if qtype == oracle.Q4_K:
        s = w["scales"].astype(np.int64)                    # (n, nsb, 12)
        sc = np.empty(s.shape[:2] + (8,), np.int64)
        mn = np.empty_like(sc)
        for i in range(4):                                  # llama_reference.cpp:116-121
            sc[..., i] = s[..., i] & 63
            sc[..., i + 4] = (s[..., i + 8] & 15) | ((s[..., i] >> 6) << 4)
            mn[..., i] = s[..., i + 4] & 63
            mn[..., i + 4] = (s[..., i + 8] >> 4) | ((s[..., i + 4] >> 6) << 4)
        qs = w["qs"].astype(np.int64).reshape(n, -1, 4, 32)  # qs[p*32 + j]
        q = np.stack([qs & 15, qs >> 4], axis=3).reshape(n, -1, 8, 32)  # sub-block 2p (low), 2p+1 (high)
        d = oracle.fp16_to_fp32(w["d"]).astype(np.float64)
        dmin = oracle.fp16_to_fp32(w["dmin"]).astype(np.float64)
        return (d[..., None, None] * sc[..., None] * q + dmin[..., None, None] * mn[..., None]).reshape(n, k)
    grid = iq2_grid_bytes().astype(np.int64)
    b = np.ascontiguousarray(w["qs"]).view(np.uint8).reshape(n, -1, 8, 8).astype(np.int64)  # (n, nsb, sub-block, byte)
    aux = b[..., 4] | (b[..., 5] << 8) | (b[..., 6] << 16) | (b[..., 7] << 24)
    scale = 2 * (aux >> 28) + 1
    v = grid[b[..., :4]]                                    # (n, nsb, 8, 4, 8) magnitudes
    d = oracle.fp16_to_fp32(w["d"]).astype(np.float64) * 0.125
    return (d[..., None, None, None] * scale[..., None, None] * v).reshape(n, k)


def unit_ratio_bound(oracle, qtype: int, w: np.ndarray, q: np.ndarray, e: np.ndarray, k: int,
                     g: np.ndarray, h: np.ndarray) -> np.ndarray:
    """Per output (m, n): sum over K of |term| in units of the smallest power
    of two every term of that output is a multiple of,
    2**(base_w + base_a + g[n] + h[m]) (times 0.125 for iq2_xxs)."""
    wmag = _weight_magnitudes(oracle, qtype, w, k)
    qk = 32 if qtype == 0 else 256
    amag = np.abs(q.astype(np.float64)) * np.repeat(_pow2(e), qk, axis=1)
    unit = _pow2(_BASE_W[qtype] + _BASE_A + g[None, :] + h[:, None]) * (0.125 if qtype == oracle.IQ2_XXS else 1.0)
    return (amag @ wmag.T) / unit


def exact_case(oracle, qtype: int, m: int, n: int, k: int, seed: int):
    """(x fp32 (m, k), aq q8 blocks, w weight blocks, r, bound) with the
    exactness precondition checked: r is the largest of 127, 63, ... 3 (with
    full weight payloads, then down to 1 with narrowed ones) that keeps every
    output's bound below 2**24, and bound is the largest one. The q8 blocks
    are the oracle's quantization of x and carry exactly the constructed
    integers and power-of-two scales."""
    rng = np.random.default_rng(seed)
    nb = k // oracle.QK[qtype]
    f = rng.integers(0, 2, nb)
    g = rng.integers(0, 2, n)
    h = rng.integers(0, 2, m)
    for narrow, rs in ((False, (127, 63, 31, 15, 7, 3)), (True, (127, 63, 31, 15, 7, 3, 1))):
        w = exact_weights(oracle, qtype, n, k, f, g, np.random.default_rng((seed, narrow)), narrow)
        for r in rs:
            x, q, e = exact_activation_rows(qtype, m, k, r, f, h, np.random.default_rng((seed, r)))
            bound = unit_ratio_bound(oracle, qtype, w, q, e, k, g, h).max()
            if bound < LIMIT:
                break
        else:
            continue
        break
    else:
        raise AssertionError("no activation range keeps the sums exact")
    aq = oracle.quantize_activation(qtype, x)
    assert np.array_equal(aq["qs"].reshape(m, k), q)
    da = oracle.fp16_to_fp32(aq["d"]) if qtype == oracle.Q4_0 else aq["d"]
    assert np.array_equal(da.astype(np.float64), _pow2(e))
    return x, aq, w, r, bound


def exact_from_isums(oracle, qtype: int, w: np.ndarray, aq: np.ndarray, isums: np.ndarray) -> np.ndarray:
    """The output from the integer block sums in float64 (exact for these
    inputs): q4_0 sum_b isum*dw*da, q4_K sum_b ad*(d*IS - dmin*IM), iq2_xxs
    sum_b 0.125*d*ad*isum."""
    if qtype == oracle.Q4_0:
        dw = oracle.fp16_to_fp32(w["d"]).astype(np.float64)
        da = oracle.fp16_to_fp32(aq["d"]).astype(np.float64)
        return np.einsum("mnb,nb,mb->mn", isums.astype(np.float64), dw, da)
    ad = aq["d"].astype(np.float64)
    d = oracle.fp16_to_fp32(w["d"]).astype(np.float64)
    if qtype == oracle.Q4_K:
        dmin = oracle.fp16_to_fp32(w["dmin"]).astype(np.float64)
        s = isums.astype(np.float64)
        return np.einsum("mnb,mb->mn", d[None] * s[..., 0] - dmin[None] * s[..., 1], ad)
    return np.einsum("mnb,nb,mb->mn", isums.astype(np.float64), 0.125 * d, ad)
