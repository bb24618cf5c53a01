"""Pins of the oracle's router matmul (engine/kernels/fn.hip:251-277, fn::f32_gemv) by what fixes it
independently of the oracle's own code:

- the step arithmetic t = fma(a.w,b.w, fma(a.z,b.z, fma(a.x,b.x, a.y*b.y))) is the order the
  reference's hipcc build emits for `acc += a.x*b.x + a.y*b.y + a.z*b.z + a.w*b.w` (compiled from
  fn.hip at -O3 for its gfx1151 target: v_mul of the y components, then v_fmac of x, z and w, then
  v_add into the accumulator); the expected values are computed here with the C library's fmaf, on
  inputs where the other orders give other bits;
- the lane partition (lane l owns float4 steps 4l + 128k) and the xor-butterfly sum, from planted
  values whose tree sum differs from a sequential sum;
- exact integer dot products, and the double-precision closed form.
"""
import ctypes
import ctypes.util

import numpy as np

import oracle

_libm = ctypes.CDLL(ctypes.util.find_library("m"))
_libm.fmaf.restype = ctypes.c_float
_libm.fmaf.argtypes = [ctypes.c_float] * 3


def fmaf(a, b, c):
    return np.float32(_libm.fmaf(float(a), float(b), float(c)))


def test_step_contraction_order():
    g = np.random.default_rng(3)
    differs = 0
    for _ in range(200):
        a = (1 + g.integers(-2 ** 12, 2 ** 12, 4) / 2.0 ** 13).astype(np.float32)
        b = (1 + g.integers(-2 ** 12, 2 ** 12, 4) / 2.0 ** 13).astype(np.float32)
        W = a.reshape(1, 4)
        x = b.reshape(1, 4)
        got = oracle.f32_gemv(W, x)[0, 0]
        want = fmaf(a[3], b[3], fmaf(a[2], b[2], fmaf(a[0], b[0], np.float32(a[1] * b[1]))))
        assert got == want
        other = fmaf(a[3], b[3], fmaf(a[2], b[2], fmaf(a[1], b[1], np.float32(a[0] * b[0]))))
        plain = np.float32(np.float32(np.float32(a[0] * b[0]) + np.float32(a[1] * b[1])) + np.float32(a[2] * b[2])) + np.float32(a[3] * b[3])
        differs += (other != want) or (plain != want)
    assert differs > 20          # the inputs do tell the orders apart


def test_lane_partition_and_tree():
    # x = 1: lane partials are W's entries.  Lane 0 (element 0) = 1, lanes 1 and 17 (elements 4 and 68)
    # = 2^-24: the tree adds lanes 1 and 17 first (1 ^ 16 = 17) -> 1 + 2^-23; in index order it stays 1
    K = 128
    W = np.zeros((1, K), np.float32)
    W[0, 0], W[0, 4], W[0, 68] = 1.0, 2.0 ** -24, 2.0 ** -24
    assert oracle.f32_gemv(W, np.ones((1, K), np.float32))[0, 0] == np.float32(1 + 2.0 ** -23)
    # the same two small values in one lane (elements 4 and 132: lane 1, steps 0 and 1) are added to
    # that lane's partial in order (2^-23), which then survives against lane 0 as well
    K = 256
    W = np.zeros((1, K), np.float32)
    W[0, 0], W[0, 4], W[0, 132] = 1.0, 2.0 ** -24, 2.0 ** -24
    assert oracle.f32_gemv(W, np.ones((1, K), np.float32))[0, 0] == np.float32(1 + 2.0 ** -23)
    # ... while elements 4 and 8 are lanes 1 and 2, which meet lane 0 separately: 1
    W = np.zeros((1, K), np.float32)
    W[0, 0], W[0, 4], W[0, 8] = 1.0, 2.0 ** -24, 2.0 ** -24
    assert oracle.f32_gemv(W, np.ones((1, K), np.float32))[0, 0] == np.float32(1.0)


def test_exact_and_closed_form():
    g = np.random.default_rng(4)
    W = g.integers(-50, 50, (33, 516)).astype(np.float32)
    x = g.integers(-50, 50, (3, 516)).astype(np.float32)
    assert np.array_equal(oracle.f32_gemv(W, x), (x.astype(np.int64) @ W.T.astype(np.int64)).astype(np.float32))
    W = g.standard_normal((65, 2560)).astype(np.float32)
    x = g.standard_normal((5, 2560)).astype(np.float32)
    ref = x.astype(np.float64) @ W.T.astype(np.float64)
    mag = np.abs(x.astype(np.float64)) @ np.abs(W.T.astype(np.float64))
    assert np.max(np.abs(oracle.f32_gemv(W, x) - ref) / mag) < 1e-6
