"""Pins of the LM-head oracle (oracle/q4k_oracle.c oq_lm_head, oracle/glm_oracle.py
bf16_dot7_rows / lm_argmax) against what the mathematics fixes.

The reference's own test of this datapath (test/glm_matmul_pipe_tb.v) checks against an
fp64 sum with a K-scaled tolerance, so there are no bit-level golden vectors to import.
The order of tools/glm_model_q4k_ref.py:476-486 (7 round-robin partial sums, then a fixed
add tree) is pinned here by cases whose exact result is derived by hand and which a
different order (sequential, another interleave width, another tree) gets wrong; products
and term coverage by exact-integer sums; the magnitude by a rigorous fp32 error bound
around the fp64 dot product; the argmax by closed-form cases of bf16_gt (:138-148) and
the scan of :826-834.  The C and numpy restatements are also checked equal.
"""
import numpy as np
import pytest

from oracle import c_oracle as co
from oracle import glm_oracle as go
from oracle import q4k_oracle as qo


def _bits(vals):
    return qo.bf16_round_bits(np.asarray(vals, np.float32))


def _dot(x, w):
    return co.bf16_dot7(_bits(x), _bits(w))


def test_dot7_exact_integer_sums():
    """Small integers: every partial sum is exact, so the result is bf16(exact dot)."""
    rng = np.random.default_rng(1)
    for K in (1, 5, 6, 7, 8, 13, 56, 200, 600):
        x = rng.integers(-15, 16, K)
        w = rng.integers(-15, 16, K)
        exact = int(np.dot(x.astype(np.int64), w.astype(np.int64)))
        b, s = _dot(x, w)
        assert float(s) == float(exact), (K, s, exact)
        assert b == qo.bf16_round_bits(np.float32(exact)), K


def test_dot7_interleave_order():
    """2^30 at k=0, -2^30 at k=7 (same partial sum, they cancel exactly), 1 at k=1 (its own
    partial sum): the 7-way order gives exactly 1.  Summed left to right the 1 is absorbed
    by 2^30 (spacing 128 there) and the result is 0."""
    x = np.ones(14, np.float32)
    w = np.zeros(14, np.float32)
    w[0], w[7], w[1] = 2.0 ** 30, -(2.0 ** 30), 1.0
    b, s = _dot(x, w)
    assert float(s) == 1.0 and b == 0x3F80
    acc = np.float32(0.0)
    for k in range(14):
        acc = np.float32(acc + np.float32(x[k] * w[k]))
    assert float(acc) == 0.0


def test_dot7_tree_order():
    """K = 7, x = 1, so the partial sums are the weights themselves.
    (2^30, 1, -2^30, 1, 1, 0, 0): ((2^30 + 1) + (-2^30 + 1)) + ((1 + 0) + (0 + 0)) = 0 + 1 = 1,
    where a left-to-right sum of the partials gives 2.
    (-2^30, 0, 0, 0, 2^30, 64, 64): (p4 + p5) = 2^30 + 64 is a tie that rounds to 2^30, then
    + (p6 + 0) = 2^30 again, so the result is -2^30 + 2^30 = 0; pairing p5 with p6 first, or
    summing left to right, gives 128."""
    b, s = _dot(np.ones(7, np.float32), [2.0 ** 30, 1.0, -(2.0 ** 30), 1.0, 1.0, 0.0, 0.0])
    assert float(s) == 1.0 and b == 0x3F80
    w2 = np.array([-(2.0 ** 30), 0.0, 0.0, 0.0, 2.0 ** 30, 64.0, 64.0], np.float32)
    b2, s2 = _dot(np.ones(7, np.float32), w2)
    assert float(s2) == 0.0 and b2 == 0x0000
    left = np.float32(0.0)
    for v in w2:
        left = np.float32(left + v)
    assert float(left) == 128.0


def test_dot7_final_rne():
    """The final rounding is bf16 RNE: 1 + 2^-8 is a tie -> 1.0; 1 + 3*2^-8 -> 1 + 2^-6."""
    b, s = _dot([1.0, 2.0 ** -8], [1.0, 1.0])
    assert float(s) == 1.0 + 2.0 ** -8 and b == 0x3F80
    b, s = _dot([1.0, 2.0 ** -8, 2.0 ** -7], [1.0, 1.0, 1.0])
    assert b == 0x3F82


def test_dot7_error_bound_vs_fp64():
    """|bf16 result - exact| <= 2^-8 |s| + (K-1) 2^-24 sum|a w| (fp32 recursive-sum bound
    plus half a bf16 ulp) on random data: a dropped term or a wrong product fails."""
    rng = np.random.default_rng(2)
    for K in (1, 7, 8, 200, 1000, 6144):
        for _ in range(4):
            xb = qo.random_bf16(rng, K)
            wb = qo.random_bf16(rng, K)
            b, s = co.bf16_dot7(xb, wb)
            xf = qo.bf16_bits_to_f32(xb).astype(np.float64)
            wf = qo.bf16_bits_to_f32(wb).astype(np.float64)
            exact = float(np.dot(xf, wf))
            mag = float(np.abs(xf * wf).sum())
            assert abs(float(s) - exact) <= max(K - 1, 0) * 2.0 ** -24 * mag * 1.0001, K
            got = float(qo.bf16_bits_to_f32(b))
            assert abs(got - float(s)) <= 2.0 ** -8 * abs(float(s)) * 1.0001, K


def test_c_equals_numpy_restatement():
    rng = np.random.default_rng(3)
    for V, K in ((5, 1), (9, 7), (33, 64), (70, 300)):
        w = qo.random_bf16(rng, (V, K))
        x = qo.random_bf16(rng, K)
        w[0, : min(K, 3)] = [0x7F80, 0xFF80, 0x0001][: min(K, 3)]   # inf, -inf, subnormal
        lc, ac = co.lm_head(w, x)
        ln, _ = go.bf16_dot7_rows(w, x)
        np.testing.assert_array_equal(lc, ln)
        assert ac == go.lm_argmax(ln)


ARGMAX_CASES = [
    # (logit bf16 patterns, expected index) -- bf16_gt and the scan, derived by hand
    ([0x3F80, 0x4000, 0x4000, 0x3F80], 1),          # tie at the max -> lower index
    ([0xFF80, 0xFF80, 0xFF80], 0),                  # all -inf: nothing beats the start
    ([0xFF80, 0xFF80, 0xBF80], 2),                  # -1 > -inf
    ([0x0000, 0x8000], 0),                          # +0 == -0
    ([0x8000, 0x0000], 0),
    ([0xBF80, 0x8000, 0x0000], 1),                  # -0 beats -1, +0 ties it
    ([0x3F80, 0x7FC0], 1),                          # +nan orders above everything
    ([0x7F80, 0x7FC0, 0x7F81], 1),                  # +nan by magnitude: 0x7FC0 > 0x7F81
    ([0xFFC0], 0),                                  # -nan orders below -inf
    ([0xFFC0, 0xFF80, 0xC0A0], 2),
    ([0xC000, 0xBF80, 0xC040], 1),                  # negatives: smaller magnitude wins
    ([0x0001, 0x0002, 0x0001], 1),                  # bf16 subnormals
]


@pytest.mark.parametrize("logits,expect", ARGMAX_CASES)
def test_argmax_closed_form(logits, expect):
    assert go.lm_argmax(np.array(logits, np.uint16)) == expect


def test_bf16_gt_c_equals_python_and_is_a_strict_order():
    rng = np.random.default_rng(4)
    pats = np.concatenate([[0, 0x8000, 0x7F80, 0xFF80, 0x7FC0, 0xFFC0, 0x7F81, 1, 0x8001], rng.integers(0, 65536, 111)])
    for a in pats:
        for b in pats:
            g = go.bf16_gt(int(a), int(b))
            assert g == co.bf16_gt(int(a), int(b))
            assert not (g and go.bf16_gt(int(b), int(a)))


def test_lm_head_sub_range_and_argmax_full():
    rng = np.random.default_rng(5)
    w = qo.random_bf16(rng, (40, 24))
    x = qo.random_bf16(rng, 24)
    full, am = co.lm_head(w, x)
    part, _ = co.lm_head(w, x, 10, 30)
    np.testing.assert_array_equal(part[10:30], full[10:30])
    assert am == go.lm_argmax(full)
