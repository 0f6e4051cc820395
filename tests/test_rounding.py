"""The q8 quantizers' rounding (device_common.h, round_half_away_q8):
(int)trunc(t + copysign(0.5 - 2^-25, t)) must equal (int)roundf(t), the
reference's rounding (llama_reference.cpp:49, :63: std::round, half away from
zero), for every value the quantizers produce (|t| <= 127 up to rounding).

Checked exhaustively here for every float32 in [0, 130] (both sides are odd
functions of t), in float32 arithmetic for the sum (numpy's IEEE round to
nearest even, as the GPU's v_add_f32) and float64 for the reference rounding.
The constant's role shows in the planted checks: with 0.5 itself, 0.5 - 2^-25
rounds up to 1."""
from __future__ import annotations

import numpy as np

HALF_MINUS = np.float32(0.49999997)  # 0x3EFFFFFF = 0.5 - 2^-25


def trick(t: np.ndarray) -> np.ndarray:
    return np.trunc((t + np.copysign(HALF_MINUS, t)).astype(np.float32)).astype(np.int64)


def round_away(t: np.ndarray) -> np.ndarray:
    a = np.abs(t.astype(np.float64))
    return (np.sign(t) * np.floor(a + 0.5)).astype(np.int64)


def test_constant_is_half_minus_2_pow_25():
    assert HALF_MINUS.view(np.uint32) == 0x3EFFFFFF
    assert float(HALF_MINUS) == 0.5 - 2.0 ** -25


def test_trick_equals_round_half_away_for_every_float_up_to_130():
    # non-negative t only: floor(t) and t - floor(t) are exact in float32, so
    # round-half-away is floor(t) + (t - floor(t) >= 0.5) without float64
    end = int(np.float32(130.0).view(np.uint32))
    step = 1 << 24
    bits = np.empty(step, dtype=np.uint32)
    for lo in range(0, end + 1, step):
        n = min(step, end + 1 - lo)
        b = bits[:n]
        b[:] = np.arange(lo, lo + n, dtype=np.uint32)
        t = b.view(np.float32)
        fl = np.floor(t)
        ref = fl + (t - fl >= np.float32(0.5))
        got = np.trunc(t + HALF_MINUS)
        bad = np.nonzero(got != ref)[0]
        assert bad.size == 0, f"first mismatch at t={t[bad[0]]!r}"


def test_negative_side_and_ties():
    t = np.array([-0.5, -1.5, -2.5, -126.5, -0.49999997, -127.0, 0.5, 2.5, 126.5], dtype=np.float32)
    assert np.array_equal(trick(t), round_away(t))
    assert list(round_away(t)) == [-1, -2, -3, -127, 0, -127, 1, 3, 127]


def test_planted_constant_half_fails():
    """With 0.5 instead of 0.5 - 2^-25 the float32 sum 0.49999997 + 0.5 rounds
    to 1.0, so the check above would catch that constant."""
    t = np.array([np.float32(0.49999997)], dtype=np.float32)
    wrong = np.trunc((t + np.float32(0.5)).astype(np.float32)).astype(np.int64)
    assert wrong[0] == 1 and round_away(t)[0] == 0
