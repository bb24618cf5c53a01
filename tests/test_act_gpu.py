"""GPU parity of the activation producers (engine/kernels/ops.hip:79-98,111-120,131,146-151) against
the CPU oracle, through the C ABI.

Bars: the norm kernels bit-exact (residual write-back, normalised row, q8 values, scales, bf16 bits),
since the library reproduces the reference's summation order and both sides compute the scale as the
correctly rounded 1/sqrt; the silu producers use the device exp (as the reference's __expf), so q8
values may move by one quantum where the host libm's exp differs by an ulp (at most 0.1% of values)
and bf16 values by one bf16 ulp.
"""
import numpy as np
import pytest
import torch

import oracle
from hipster_amd import qmm, synth
from tests.gpu_util import dev, host

pytestmark = pytest.mark.gpu

EPS = 1e-6


def run_norm_quant(x, y, w, eps, with_ds):
    T, n = x.shape
    xd = dev(x)
    xn = torch.full((T, n), float("nan"), device="cuda")
    xq = qmm.XQ8Buf(T, n, with_ds=with_ds)
    qmm.add_rmsnorm_quant(xd, None if y is None else dev(y), dev(w), xn, xq, T, n, eps)
    return host(xd), host(xn), host(xq.q), host(xq.d), host(xq.s), None if xq.ds is None else host(xq.ds)


@pytest.mark.parametrize("T,n,has_y", [(1, 5120, True), (1, 5120, False), (7, 2560, True), (64, 5120, True),
                                       (2, 32, True), (3, 6144, True), (2, 6176, True), (2, 16384, False),
                                       (5, 1056, True), (2048, 5120, True)])
def test_add_rmsnorm_quant_bit_exact(gpu, T, n, has_y):
    print(f"add_rmsnorm_quant T={T} n={n} y={has_y}", flush=True)
    x = synth.normal_f32(700 + n + T, (T, n)) * 2
    y = synth.normal_f32(701 + n + T, (T, n)) if has_y else None
    w = synth.normal_f32(702 + n, (n,)) * 0.3 + 1
    if T > 1:
        x[1] = 0.0                               # an all-zero row (scale 1/sqrt(eps), q = 0)
        if has_y:
            y[1] = 0.0
    xs, xn, q, d, s, ds = run_norm_quant(x, y, w, EPS, with_ds=(T == 7))
    xs_r, xn_r, q_r, d_r, s_r = oracle.add_rmsnorm_quant(x, y, w, EPS)
    assert np.array_equal(xs, xs_r)
    assert np.array_equal(xn.view(np.uint32), xn_r.view(np.uint32)), int((xn != xn_r).sum())
    assert np.array_equal(q, q_r)
    assert np.array_equal(d.view(np.uint32), d_r.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), s_r.view(np.uint32))
    if ds is not None:
        assert np.array_equal(ds[..., 0], d_r) and np.array_equal(ds[..., 1], s_r)


@pytest.mark.parametrize("T,n,has_y", [(1, 5120, True), (9, 2560, False), (2048, 5120, True), (3, 100, True),
                                       (2, 7000, True), (1, 16384, True), (4, 1, False)])
def test_add_rmsnorm_bf16_bit_exact(gpu, T, n, has_y):
    print(f"add_rmsnorm_bf16 T={T} n={n} y={has_y}", flush=True)
    x = synth.normal_f32(720 + n + T, (T, n)) * 2
    y = synth.normal_f32(721 + n + T, (T, n)) if has_y else None
    w = synth.normal_f32(722 + n, (n,)) * 0.3 + 1
    xd = dev(x)
    xb = torch.full((T, n), -1, dtype=torch.int16, device="cuda")
    qmm.add_rmsnorm_bf16(xd, None if y is None else dev(y), dev(w), xb, T, n, EPS)
    xs_r, xb_r = oracle.add_rmsnorm_bf16(x, y, w, EPS)
    assert np.array_equal(host(xd), xs_r)
    assert np.array_equal(host(xb).view(np.uint16), xb_r)


@pytest.mark.parametrize("n", [5120, 1056])
def test_add_rmsnorm_unaligned_rows(gpu, n):
    """Rows that are not 16-byte aligned take the one-value-per-lane layout: the same bits."""
    T = 5
    x = synth.normal_f32(780 + n, (T, n)); y = synth.normal_f32(781 + n, (T, n)); w = synth.normal_f32(782 + n, (n,)) + 1

    def view(a):                             # a device copy that starts one float past a 256-byte boundary
        buf = torch.zeros(a.size + 1, device="cuda")
        buf[1:] = dev(a.reshape(-1))
        return buf[1:]

    xd, yd, wd = view(x), view(y), view(w)
    xn = torch.zeros(T * n + 1, device="cuda")[1:]
    xq = qmm.XQ8Buf(T, n)
    qmm.add_rmsnorm_quant(xd, yd, wd, xn, xq, T, n, EPS)
    xs_r, xn_r, q_r, d_r, s_r = oracle.add_rmsnorm_quant(x, y, w, EPS)
    assert np.array_equal(host(xd).reshape(T, n), xs_r)
    assert np.array_equal(host(xn).reshape(T, n).view(np.uint32), xn_r.view(np.uint32))
    assert np.array_equal(host(xq.q), q_r) and np.array_equal(host(xq.d), d_r) and np.array_equal(host(xq.s), s_r)
    xd2 = view(x)
    xb = torch.zeros(T * n + 1, dtype=torch.int16, device="cuda")[1:]
    qmm.add_rmsnorm_bf16(xd2, yd, wd, xb, T, n, EPS)
    _, xb_r = oracle.add_rmsnorm_bf16(x, y, w, EPS)
    assert np.array_equal(host(xb).reshape(T, n).view(np.uint16), xb_r)


def test_add_rmsnorm_quant_and_bf16_agree(gpu):
    """Both kernels own the same elements per thread, so the bf16 row is RNE of the q8 kernel's xn."""
    T, n = 16, 5120
    x = synth.normal_f32(730, (T, n)); y = synth.normal_f32(731, (T, n)); w = synth.normal_f32(732, (n,)) + 1
    _, xn, _, _, _, _ = run_norm_quant(x, y, w, EPS, False)
    xb = torch.zeros((T, n), dtype=torch.int16, device="cuda")
    qmm.add_rmsnorm_bf16(dev(x), dev(y), dev(w), xb, T, n, EPS)
    assert np.array_equal(host(xb).view(np.uint16), synth.to_bf16_bits(xn))


def test_add_rmsnorm_quant_row_independent(gpu):
    """A row's outputs do not depend on the other rows of the batch."""
    T, n = 33, 5120
    x = synth.normal_f32(740, (T, n)); y = synth.normal_f32(741, (T, n)); w = synth.normal_f32(742, (n,)) + 1
    _, xn_all, q_all, _, _, _ = run_norm_quant(x, y, w, EPS, False)
    _, xn_one, q_one, _, _, _ = run_norm_quant(x[17:18].copy(), y[17:18].copy(), w, EPS, False)
    assert np.array_equal(xn_all[17], xn_one[0]) and np.array_equal(q_all[17], q_one[0])


@pytest.mark.parametrize("n,off", [(32, 0), (17408, 0), (2048 * 17408 // 16, 0), (17408, 1)])
def test_silu_mul_quant(gpu, n, off):
    """off = 1 passes 4-byte-aligned views of g and u, which take the one-value-per-lane kernel."""
    print(f"silu_mul_quant n={n} off={off}", flush=True)
    g = synth.normal_f32(750 + n % 97, (n,)) * 3
    u = synth.normal_f32(751 + n % 97, (n,))
    g[:32] = 0.0
    xq = qmm.XQ8Buf(1, n, with_ds=True)
    gd = torch.zeros(n + off, device="cuda"); ud = torch.zeros(n + off, device="cuda")
    gd[off:] = dev(g); ud[off:] = dev(u)
    qmm.silu_mul_quant(gd[off:], ud[off:], xq, n)
    h = np.empty_like(g)
    oracle.lib().qo_silu_mul(oracle._ptr(g), oracle._ptr(u), g.size, oracle._ptr(h))
    q, d, s = oracle.quantize_x_q8(h)
    gq, gd, gds = host(xq.q), host(xq.d), host(xq.ds)
    assert np.max(np.abs(gq.astype(int) - q.astype(int))) <= 1
    assert np.mean(gq != q) < 1e-3
    np.testing.assert_allclose(gd, d, rtol=1e-5)
    assert np.array_equal(gds[..., 0], gd) and np.array_equal(gds[..., 1], host(xq.s))
    assert not gq[0, :32].any() and gd[0, 0] == 0.0


@pytest.mark.parametrize("rows", [11, 2048])
def test_silu_mul_quant_equals_moe_silu_quant(gpu, rows):
    """ops.hip:146-151 and fn.hip:206-211 are the same arithmetic (and amax, sum(q) are exact in any
    order): the four-values-per-lane kernel gives bit for bit the one-value-per-lane kernel's q8."""
    n = 512
    g = dev(synth.normal_f32(760, (rows, n)) * 3); u = dev(synth.normal_f32(761, (rows, n)))
    g[0, 64:96] = 0.0
    a = qmm.XQ8Buf(rows, n); b = qmm.XQ8Buf(rows, n)
    qmm.silu_mul_quant(g, u, a, rows * n)
    qmm.moe_silu_quant(g, u, b, rows, n)
    for t1, t2 in ((a.q, b.q), (a.d, b.d), (a.s, b.s)):
        assert torch.equal(t1, t2)


@pytest.mark.parametrize("n,off", [(17408, 0), (1000003, 0), (4099, 1)])
def test_silu_mul_bf16(gpu, n, off):
    """out = bf16(silu(g)*u); the misaligned view (off=1) takes the per-element path."""
    print(f"silu_mul_bf16 n={n} off={off}", flush=True)
    g = synth.normal_f32(770 + off, (n + off,)) * 3
    u = synth.normal_f32(771 + off, (n + off,))
    gd, ud = dev(g)[off:], dev(u)[off:]
    out = torch.full((n + off,), -1, dtype=torch.int16, device="cuda")[off:]
    qmm.silu_mul_bf16(gd, ud, out, n)
    gh, uh = g[off:].copy(), u[off:].copy()          # kept alive across the ctypes call
    h = np.empty(n, np.float32)
    oracle.lib().qo_silu_mul(oracle._ptr(gh), oracle._ptr(uh), n, oracle._ptr(h))
    ref = synth.to_bf16_bits(h).astype(np.int32)
    got = host(out).view(np.uint16).astype(np.int32)
    diff = np.abs(got - ref)
    assert diff.max() <= 1 and np.mean(diff != 0) < 1e-3
    # and bit for bit the bf16 path of the MoE (the same arithmetic, fn.hip:206-211)
    h2 = torch.zeros(n, dtype=torch.int16, device="cuda")
    qmm.moe_silu_bf16(gd, ud, h2, n)
    assert torch.equal(out, h2)
