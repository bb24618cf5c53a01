"""Pins of the oracle's activation producers (engine/kernels/ops.hip:62-120,146-151) by what the
mathematics fixes, not by restating the oracle's formula:

- the reduction tree of block_sum1024 (ops.hip:64-78) from inputs whose tree sum differs from the
  sequential sum and from any other pairing, worked out by hand;
- the normalised row against the closed form x * w / sqrt(mean(x^2) + eps) in double;
- exact special cases (constant rows, power-of-two scaling, y = None vs y = 0, the residual
  write-back);
- the quantised output equal to the q8 quantiser (pinned against the reference's golden vectors in
  test_oracle.py) applied to the normalised row, and the bf16 output equal to the RNE rounding of
  the same row.
"""
import numpy as np
import pytest

import oracle
from hipster_amd import synth

EPS = 1e-6


def closed_form(x, w, eps):
    x = np.asarray(x, np.float64)
    return x * np.asarray(w, np.float64) / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def test_block_sum_pairs_lane_l_with_l_xor_16_first():
    # inside one group of 32: 1 + 2^-24 + 2^-24 summed in index order stays 1 (each 2^-24 is a tie
    # that rounds to even), but the butterfly adds lanes 1 and 17 first (1 ^ 16 == 17), giving 2^-23
    # that survives: 1 + 2^-23.
    p = np.zeros(1024, np.float32)
    p[0], p[1], p[17] = 1.0, 2.0 ** -24, 2.0 ** -24
    assert oracle.block_sum1024(p) == np.float32(1.0 + 2.0 ** -23)
    # lanes 1 and 2 are never paired with each other before one of them meets lane 0: lane 2 joins
    # lane 0 at step o=2 (1 + 2^-24 -> 1), lane 1 at step o=1 (1 + 2^-24 -> 1); a tree pairing 1
    # with 2 first would give 1 + 2^-23
    p = np.zeros(1024, np.float32)
    p[0], p[1], p[2] = 1.0, 2.0 ** -24, 2.0 ** -24
    assert oracle.block_sum1024(p) == np.float32(1.0)


def test_block_sum_second_stage_is_the_same_tree_over_group_sums():
    # group sums g[0] = 1, g[1] = g[17] = 2^-24 (one value per group in lane 0)
    p = np.zeros(1024, np.float32)
    p[0], p[32 * 1], p[32 * 17] = 1.0, 2.0 ** -24, 2.0 ** -24
    assert oracle.block_sum1024(p) == np.float32(1.0 + 2.0 ** -23)
    p = np.zeros(1024, np.float32)
    p[0], p[32 * 1], p[32 * 2] = 1.0, 2.0 ** -24, 2.0 ** -24
    assert oracle.block_sum1024(p) == np.float32(1.0)


def test_block_sum_exact_on_integers_and_close_on_random():
    g = np.random.default_rng(5)
    p = g.integers(-1000, 1000, 1024).astype(np.float32)
    assert oracle.block_sum1024(p) == float(p.astype(np.int64).sum())
    p = g.standard_normal(1024).astype(np.float32)
    assert abs(oracle.block_sum1024(p) - float(np.sum(p.astype(np.float64)))) < 1e-4


@pytest.mark.parametrize("T,n", [(1, 5120), (3, 2560), (2, 32), (1, 6144), (2, 8192), (1, 16384), (1, 1056)])
def test_add_rmsnorm_matches_closed_form(T, n):
    x = synth.normal_f32(600 + n, (T, n)) * 3
    y = synth.normal_f32(601 + n, (T, n))
    w = synth.normal_f32(602 + n, (n,)) * 0.2 + 1
    xs, xn, q, d, s = oracle.add_rmsnorm_quant(x, y, w, EPS)
    assert np.array_equal(xs, x + y)                               # residual add, written back
    ref = closed_form(x + y, w, EPS)
    assert np.max(np.abs(xn - ref) / (np.abs(ref) + 1e-3)) < 2e-6
    # xq is the reference-pinned q8 quantiser of the normalised row
    q2, d2, s2 = oracle.quantize_x_q8(xn)
    assert np.array_equal(q, q2) and np.array_equal(d, d2) and np.array_equal(s, s2)
    # bf16 variant: the same scale (same sum, same tree), so xb is RNE of the same row
    xs_b, xb = oracle.add_rmsnorm_bf16(x, y, w, EPS)
    assert np.array_equal(xs_b, xs)
    assert np.array_equal(xb, synth.to_bf16_bits(xn))


def test_add_rmsnorm_exact_special_cases():
    n = 4096
    # a row of ones, eps 0: mean square exactly 1, scale exactly 1, xn == w
    w = synth.normal_f32(610, (n,))
    _, xn, _, _, _ = oracle.add_rmsnorm_quant(np.ones((1, n), np.float32), None, w, 0.0)
    assert np.array_equal(xn[0], w)
    # scaling x by 2 scales every partial square by 4 exactly and the scale by 1/2 exactly (eps 0)
    x = synth.normal_f32(611, (2, n))
    _, xn1, q1, d1, _ = oracle.add_rmsnorm_quant(x, None, w, 0.0)
    _, xn2, q2, d2, _ = oracle.add_rmsnorm_quant(2 * x, None, w, 0.0)
    assert np.array_equal(xn1, xn2) and np.array_equal(q1, q2) and np.array_equal(d1, d2)
    # y = None is the same as y = 0 (and leaves x as it was)
    a = oracle.add_rmsnorm_quant(x, None, w, EPS)
    b = oracle.add_rmsnorm_quant(x, np.zeros_like(x), w, EPS)
    for u, v in zip(a, b):
        assert np.array_equal(u, v)
    assert np.array_equal(a[0], x)
    # eps enters as mean + eps: an all-zero row gives xn = 0 (scale 1/sqrt(eps), finite)
    _, xn0, q0, d0, s0 = oracle.add_rmsnorm_quant(np.zeros((1, 64), np.float32), None, np.ones(64, np.float32), EPS)
    assert not xn0.any() and not q0.any() and not d0.any() and not s0.any()
    # eps is not dropped: for a tiny row, eps dominates the mean square
    xt = np.full((1, 64), 1e-4, np.float32)
    _, xnt, _, _, _ = oracle.add_rmsnorm_quant(xt, None, np.ones(64, np.float32), 1e-2)
    assert np.allclose(xnt, 1e-4 / np.sqrt(1e-8 + 1e-2), rtol=1e-6)


def test_add_rmsnorm_shape_errors():
    w = np.ones(48, np.float32)
    with pytest.raises(ValueError):
        oracle.add_rmsnorm_quant(np.ones((1, 48), np.float32), None, w, EPS)   # n % 32 != 0
    _, xb = oracle.add_rmsnorm_bf16(np.ones((1, 48), np.float32), None, w, EPS)  # the bf16 form takes any n
    assert np.array_equal(xb, synth.to_bf16_bits(np.full((1, 48), 1 / np.sqrt(1 + EPS), np.float32)))
