"""CPU: the oracle's restatement of the tied output head's dot product
(crates/llm-core/src/ops/linear.rs:19-32 `dot`, :110-125 `linear_fwd`).

Pinned by closed forms, none of which retypes the oracle's loop:
  * one-hot rows: y[o] = w[o][j] exactly;
  * small integers: every product and partial sum is exact, so y is the
    integer dot product;
  * rows whose values are chosen so that the reference's order (four
    strided accumulators, then (acc0 + acc1) + (acc2 + acc3), then the
    remainder) gives a different binary32 result than a sequential fold, a
    pairwise tree, contiguous quarters, or the remainder folded into the
    accumulators. The expected values are worked out by hand below;
  * random rows: within the f32 error bound of the exact (float64) dot
    product, and x @ w^T rather than a transposed operand.
"""
import numpy as np
import pytest

from oracle import oracle

T24 = float(2 ** 24)


def test_one_hot_rows_pick_the_weight_column():
    rs = np.random.default_rng(1)
    for in_dim in (4, 7, 64, 257):
        w = rs.standard_normal((33, in_dim)).astype(np.float32)
        x = np.eye(in_dim, dtype=np.float32)
        y = oracle.linear_fwd(x, w)
        assert np.array_equal(y, w.T)


def test_small_integers_are_exact():
    rs = np.random.default_rng(2)
    for in_dim in (1, 3, 4, 5, 16, 130, 512):
        x = rs.integers(-8, 9, size=(5, in_dim))
        w = rs.integers(-8, 9, size=(40, in_dim))
        y = oracle.linear_fwd(x.astype(np.float32), w.astype(np.float32))
        assert np.array_equal(y, (x @ w.T).astype(np.float32))


@pytest.mark.parametrize(
    "a,expected",
    [
        # acc = [1+1, 2^24+0, 1+0, 0]: (2 + 2^24) = 2^24+2, plus (1 + 0): 2^24+3
        # is a tie between 2^24+2 (odd mantissa) and 2^24+4 (even): 2^24+4.
        # A sequential fold or a pairwise tree gives 2^24 (1 + 2^24 rounds
        # to 2^24 first), contiguous quarters give 2^24 as well.
        ([1.0, T24, 1.0, 0.0, 1.0, 0.0, 0.0, 0.0], T24 + 4),
        # acc = [2^24, 0, 1, 1]: (2^24 + 0) + (1 + 1) = 2^24 + 2 exactly; a
        # sequential fold of a gives ((2^24 + 1) + 1) = 2^24.
        ([T24, 0.0, 1.0, 1.0], T24 + 2),
        # four accumulators give 2^24, the remainder 1+1+1 = 3 is added last:
        # 2^24 + 3 -> 2^24 + 4 (tie to even). Folding the remainder into the
        # accumulators instead gives 2^24.
        ([T24, 0.0, 0.0, 0.0, 1.0, 1.0, 1.0], T24 + 4),
    ],
)
def test_summation_order(a, expected):
    x = np.array([a], dtype=np.float32)
    w = np.ones((1, len(a)), dtype=np.float32)
    y = oracle.linear_fwd(x, w)
    assert y[0, 0] == np.float32(expected)


def test_random_rows_within_the_error_bound_and_not_transposed():
    rs = np.random.default_rng(3)
    rows, in_dim, out_dim = 6, 256, 300
    x = rs.standard_normal((rows, in_dim)).astype(np.float32)
    w = (0.02 * rs.standard_normal((out_dim, in_dim))).astype(np.float32)
    y = oracle.linear_fwd(x, w, threads=4)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    bound = (in_dim / 4 + 3) * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T)
    assert np.all(np.abs(y - exact) <= bound)
    assert y.shape == (rows, out_dim)
    # threads do not change the result
    assert np.array_equal(y, oracle.linear_fwd(x, w, threads=1))
