"""CPU tests that pin the oracle's other weight formats (Q5_K, IQ4_XS, Q8_0, Q5_1, Q5_0 and the row-SoA
repacks Q8_0_SOA / Q5_1_SOA) before the GPU kernels are checked against it:
  * dequantisation bit-exact against golden vectors written by the reference's own engine/src/quant.h
    (tests/golden/make_golden.py --formats), special blocks included (zero, negative and subnormal
    scales, all-ones and all-zero quant bytes), and against the compiled reference itself on fresh
    random rows when oracle/_ref is present;
  * the load-time repacks byte-exact against the bytes the reference's own gemv.hip repacks produced
    (same file), for K = 512 and a K that is not a multiple of 256; the SoA readers by round trip
    (repacked row decodes to the golden values of the GGUF row);
  * Q5_0 -> Q5_1 SoA (m = -16 d) equal to the Q5_0 definition w = (q - 16) d, bit for bit;
  * row byte counts against the reference's wfmt_row_bytes; f32 -> f16 against numpy's RNE.
"""
import os

import numpy as np
import pytest

import oracle
from hipster_amd import synth

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "quant_golden_fmt.npz"))


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def dq_rows(fmt, W, K):
    return oracle.dequant_rows(fmt, np.ascontiguousarray(W), K)


@pytest.mark.parametrize("fmt,key", [(oracle.Q5_K, "q5k"), (oracle.IQ4_XS, "iq4xs"), (oracle.Q8_0, "q8_0"),
                                     (oracle.Q5_1, "q5_1")])
def test_dequant_matches_reference_golden(fmt, key):
    bl = G[key + "_blocks"]
    per = synth.BLOCK[fmt][0]
    y = dq_rows(fmt, bl, per)
    assert np.array_equal(bits(y), bits(G[key + "_y"]))


def test_dequant_known_answers():
    L = oracle.lib()
    # Q8_0: d = 1, q = -16..15 -> w = q
    b = np.zeros(34, np.uint8); b[0:2] = np.array([np.float16(1.0)]).view(np.uint8)
    b[2:] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    y = np.empty(32, np.float32); L.qo_dequant_q8_0_block(b.ctypes.data, y.ctypes.data)
    assert np.array_equal(y, np.arange(-16, 16, dtype=np.float32))
    # IQ4_XS: d = 1, every scale 33 (ls - 32 = 1) -> w = level[nibble]
    b = np.zeros(136, np.uint8); b[0:2] = np.array([np.float16(1.0)]).view(np.uint8)
    b[2:4] = np.array([0xAAAA], np.uint16).view(np.uint8)       # high bits 2 of every scale: 0b10 -> 32
    b[4:8] = 0x11                                               # low nibbles 1 -> ls = 33
    b[8:] = np.tile(np.array([0x10 * ((j + 3) % 16) + j for j in range(16)], np.uint8), 8)
    y = np.empty(256, np.float32); L.qo_dequant_iq4_xs_block(b.ctypes.data, y.ctypes.data)
    lv = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)
    want = np.concatenate([np.concatenate([lv[np.arange(16)], lv[(np.arange(16) + 3) % 16]])] * 8)
    assert np.array_equal(y, want)
    # Q5_1: d = 1, m = -16, qh bit j set for j in the low half only -> w = nibble + 16 - 16 / nibble - 16
    b = np.zeros(24, np.uint8); b[0:2] = np.array([np.float16(1.0)]).view(np.uint8)
    b[2:4] = np.array([np.float16(-16.0)]).view(np.uint8); b[4:8] = np.array([0x0000FFFF], np.uint32).view(np.uint8)
    b[8:] = np.array([(15 - j) * 16 + j for j in range(16)], np.uint8)
    y = np.empty(32, np.float32); L.qo_dequant_q5_1_block(b.ctypes.data, y.ctypes.data)
    assert np.array_equal(y[:16], np.arange(16, dtype=np.float32)) and np.array_equal(y[16:], np.arange(15, -1, -1) - 16.0)


def test_dequant_random_rows_vs_compiled_reference():
    ref = oracle.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    for fmt, gtype in ((oracle.Q5_K, 13), (oracle.IQ4_XS, 23), (oracle.Q8_0, 8), (oracle.Q5_1, 7)):
        K = 1024
        W = synth.matrix(777 + fmt, fmt, 50, K)
        y = dq_rows(fmt, W, K)
        r = np.empty_like(y)
        for i in range(W.shape[0]):
            row = np.ascontiguousarray(W[i])
            ref.ref_dequant_row(gtype, row.ctypes.data, r[i].ctypes.data, K)
        assert np.array_equal(bits(y), bits(r)), fmt


@pytest.mark.parametrize("name,fn,src_fmt", [("q8_0", "qo_repack_row_q8_0", oracle.Q8_0),
                                             ("q5_1", "qo_repack_row_q5_1", oracle.Q5_1),
                                             ("q5_0", "qo_repack_row_q5_0", oracle.Q5_0)])
@pytest.mark.parametrize("K", [512, 96])
def test_repack_matches_reference_bytes(name, fn, src_fmt, K):
    src, dst = G[f"repack_{name}_K{K}_src"], G[f"repack_{name}_K{K}_dst"]
    L = oracle.lib()
    for r in range(src.shape[0]):
        out = np.zeros(dst.shape[1], np.uint8)
        s = np.ascontiguousarray(src[r])
        getattr(L, fn)(s.ctypes.data, out.ctypes.data, K)
        assert np.array_equal(out, dst[r])
    # the numpy repacks of hipster_amd.synth (test and bench data) give the same bytes
    if name == "q8_0":
        assert np.array_equal(synth.repack_q8_0_soa(src, K), dst)
    elif name == "q5_1":
        assert np.array_equal(synth.repack_q5_1_soa(src, K), dst)


@pytest.mark.parametrize("K", [512, 96])
def test_soa_rows_decode_to_the_gguf_rows(K):
    for gguf, soa, rep in ((oracle.Q8_0, oracle.Q8_0_SOA, synth.repack_q8_0_soa), (oracle.Q5_1, oracle.Q5_1_SOA, synth.repack_q5_1_soa)):
        W = synth.matrix(55 + gguf, gguf, 6, K)
        assert np.array_equal(bits(dq_rows(soa, rep(W, K), K)), bits(dq_rows(gguf, W, K)))
    # and the golden rows through the reference's own repack output
    for name, gguf, soa in (("q8_0", oracle.Q8_0, oracle.Q8_0_SOA), ("q5_1", oracle.Q5_1, oracle.Q5_1_SOA)):
        src, dst = G[f"repack_{name}_K{K}_src"], G[f"repack_{name}_K{K}_dst"]
        assert np.array_equal(bits(dq_rows(soa, dst, K)), bits(dq_rows(gguf, src, K)))


def test_q5_0_repack_equals_definition():
    # finite d only (the golden rows also hold an infinite and a subnormal d for the repack bytes)
    K = 512
    W = synth.matrix(61, oracle.Q5_0, 8, K)
    L = oracle.lib()
    for r in range(W.shape[0]):
        out = np.zeros(K // 32 * 24, np.uint8)
        s = np.ascontiguousarray(W[r])
        L.qo_repack_row_q5_0(s.ctypes.data, out.ctypes.data, K)
        assert np.array_equal(bits(dq_rows(oracle.Q5_1_SOA, out[None], K)), bits(dq_rows(oracle.Q5_0, W[r:r + 1], K)))


def test_row_bytes_match_reference():
    for i, K in enumerate((256, 512, 5120, 17408)):
        for f in range(6):
            assert oracle.row_bytes(f, K) == G["row_bytes"][i, f], (f, K)


def test_f32_to_f16_matches_numpy_rne():
    L = oracle.lib()
    g = np.random.default_rng(5)
    v = np.concatenate([g.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** g.integers(-9, 5, 20000),
                        np.array([65504, 65519.99, 65520, 1e9, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 0.0, -0.0], np.float32)])
    with np.errstate(over="ignore"):
        want = v.astype(np.float16).view(np.uint16)
    got = np.array([L.qo_f32_to_f16(float(x)) for x in v], np.uint16)
    assert np.array_equal(got, want)
