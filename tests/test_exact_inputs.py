"""CPU checks of the exact-arithmetic inputs (tests/exact_inputs.py) that the
GPU tests compare bit for bit.

1. The construction holds: the oracle's fp32 output (the reference's operation
   order, llama_reference.cpp:113-161) equals the float64 value computed from
   the brute-force int64 block sums, on every output. So on these inputs the
   fp32 result does not depend on the order of the additions.
2. A planted +-1 in any one block sum changes that output's bits, so the
   bitwise comparison of the GPU tests catches an off-by-one block sum that the
   1e-5 * sum|terms| tolerance lets through.
"""
from __future__ import annotations

import numpy as np
import pytest

from exact_inputs import LIMIT, exact_case, exact_from_isums


@pytest.mark.parametrize("qtype,m,n,k", [(0, 3, 64, 4096), (0, 2, 16, 65536), (0, 17, 40, 8192),
                                         (1, 3, 64, 4096), (1, 5, 24, 8192), (2, 3, 64, 4096), (2, 4, 24, 8192)])
def test_exact_inputs_make_the_oracle_order_independent(oracle, qtype, m, n, k):
    x, aq, w, r, bound = exact_case(oracle, qtype, m, n, k, seed=m * 7 + k)
    isums = oracle.isums(qtype, w, aq, m, n, k)
    exact = exact_from_isums(oracle, qtype, w, aq, isums)
    got = oracle.matmul(qtype, w, aq, m, n, k)
    assert np.array_equal(exact.astype(np.float32).astype(np.float64), exact)  # representable in fp32
    assert np.array_equal(got.astype(np.float64), exact)
    # compute() from the fp32 rows quantizes back to the same blocks
    assert np.array_equal(oracle.compute(qtype, x, w), got)
    # the sums use a fair part of the exact range (not trivially small inputs)
    assert LIMIT / 64 < bound < LIMIT, (r, bound)


@pytest.mark.parametrize("qtype", [0, 1, 2])
def test_planted_off_by_one_block_sum_changes_the_output(oracle, qtype):
    """Plant +1 or -1 in one block sum (for q4_K in the scale sum IS or the
    min sum IM) at 200 random places: every such output differs from the
    oracle's bits."""
    m, n, k = 4, 48, 4096
    x, aq, w, _, _ = exact_case(oracle, qtype, m, n, k, seed=11 + qtype)
    isums = oracle.isums(qtype, w, aq, m, n, k)
    ref = oracle.matmul(qtype, w, aq, m, n, k)
    rng = np.random.default_rng(qtype)
    for _ in range(200):
        planted = isums.copy()
        idx = tuple(int(rng.integers(0, s)) for s in planted.shape)
        planted[idx] += 1 if rng.random() < 0.5 else -1
        wrong = exact_from_isums(oracle, qtype, w, aq, planted).astype(np.float32)
        mi, ni = idx[0], idx[1]
        assert wrong[mi, ni].view(np.uint32) != ref[mi, ni].view(np.uint32), idx
        others = np.ones((m, n), bool)
        others[mi, ni] = False
        assert np.array_equal(wrong[others], ref[others])
