"""CPU-side checks of the C ABI: the library loads, exports every function include/hipster_qmm.h
declares, the host helpers match the oracle, and argument validation returns error codes before any
device work (these calls never reach the GPU)."""
import ctypes
import os
import re

import numpy as np
import pytest

from hipster_amd import _lib, synth

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))


def header_functions():
    text = open(os.path.join(ROOT, "include", "hipster_qmm.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qmm_[a-z0-9_A-Z]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    missing = [n for n in header_functions() if not hasattr(L, n)]
    assert not missing, missing
    # and the ctypes signature table covers the header
    assert set(header_functions()) <= set(_lib.SIGNATURES), set(header_functions()) - set(_lib.SIGNATURES)


def test_version_and_status_strings():
    L = _lib.lib()
    assert b"gfx950" in L.qmm_version()
    assert L.qmm_status_string(0) == b"ok"
    assert L.qmm_status_string(-1) == b"unsupported weight format"
    for code in range(-10, 0):    # every status the header defines has its own text
        assert L.qmm_status_string(code) != b"unknown status", code
    assert L.qmm_status_string(-11) == b"unknown status"


def test_row_bytes_and_repack_match_oracle():
    L = _lib.lib()
    assert L.qmm_wfmt_row_bytes(_lib.QMM_Q4_K, 5120) == 20 * 144
    assert L.qmm_wfmt_row_bytes(_lib.QMM_Q6_K, 17408) == 68 * 210
    assert L.qmm_wfmt_row_bytes(_lib.QMM_Q6_K_SOA, 17408) == 68 * 210
    assert L.qmm_wfmt_row_bytes(_lib.QMM_Q4_K, 100) == 0
    assert L.qmm_wfmt_row_bytes(_lib.QMM_Q5_K, 100) == 0
    assert L.qmm_wfmt_row_bytes(_lib.QMM_Q8_0_SOA, 96) == 102 and L.qmm_wfmt_row_bytes(_lib.QMM_Q5_1_SOA, 96) == 72
    assert L.qmm_wfmt_row_bytes(_lib.QMM_Q8_0_SOA, 100) == 0 and L.qmm_wfmt_row_bytes(99, 256) == 0
    # every format against the reference's own wfmt_row_bytes (golden table)
    G = np.load(os.path.join(os.path.dirname(__file__), "golden", "quant_golden_fmt.npz"))
    for i, K in enumerate((256, 512, 5120, 17408)):
        for fmt in range(6):
            assert L.qmm_wfmt_row_bytes(fmt, K) == G["row_bytes"][i, fmt], (fmt, K)
    W = synth.matrix(5, synth.Q6_K, 4, 2048)
    soa = synth.repack_q6k_soa(W, 2048)
    for r in range(4):
        src = np.ascontiguousarray(W[r]); dst = np.empty_like(src)
        assert L.qmm_repack_row_q6_K(src.ctypes.data, dst.ctypes.data, 2048) == 0
        assert np.array_equal(dst, soa[r])
    assert L.qmm_repack_row_q6_K(None, None, 256) == -3


@pytest.mark.parametrize("name,fn", [("q8_0", "qmm_repack_row_q8_0"), ("q5_1", "qmm_repack_row_q5_1"),
                                     ("q5_0", "qmm_repack_row_q5_0")])
@pytest.mark.parametrize("K", [512, 96])
def test_repacks_match_reference_bytes(name, fn, K):
    """The three load-time repacks against the bytes the reference's own gemv.hip wrote (golden)."""
    G = np.load(os.path.join(os.path.dirname(__file__), "golden", "quant_golden_fmt.npz"))
    src, want = G[f"repack_{name}_K{K}_src"], G[f"repack_{name}_K{K}_dst"]
    L = _lib.lib()
    for r in range(src.shape[0]):
        s = np.ascontiguousarray(src[r]); d = np.zeros(want.shape[1], np.uint8)
        assert getattr(L, fn)(s.ctypes.data, d.ctypes.data, K) == 0
        assert np.array_equal(d, want[r])
    assert getattr(L, fn)(None, None, 32) == -3
    assert getattr(L, fn)(src.ctypes.data, src.ctypes.data, 100) == -2


def _xq(p=1):
    return _lib.XQ8(p, p, p, 0)


def test_argument_validation_without_device_work():
    L = _lib.lib()
    dummy = ctypes.c_void_p(16)
    # unknown formats are refused (the reference aborts here); the other formats check their shape
    assert L.qmm_gemv_q8(99, dummy, _xq(16), dummy, 16, 256, 1, 0, 1, None) == -1
    # K granules: 256 (block formats), 64 (Q8_0_SOA: rows dword aligned), 32 (Q5_1_SOA)
    for fmt, badk in ((_lib.QMM_Q5_K, 96), (_lib.QMM_IQ4_XS, 640), (_lib.QMM_Q8_0_SOA, 96), (_lib.QMM_Q5_1_SOA, 100)):
        assert L.qmm_gemv_q8(fmt, dummy, _xq(16), dummy, 16, badk, 1, 0, 1, None) == -2
        assert L.qmm_gemv_q8(fmt, dummy, _xq(16), dummy, 16, 256, 9, 0, 1, None) == -2
    # bad shapes
    assert L.qmm_gemv_q8(_lib.QMM_Q4_K, dummy, _xq(16), dummy, 16, 300, 1, 0, 1, None) == -2
    assert L.qmm_gemv_q8(_lib.QMM_Q4_K, dummy, _xq(16), dummy, 0, 256, 1, 0, 1, None) == -2
    assert L.qmm_gemv_q8(_lib.QMM_Q4_K, dummy, _xq(16), dummy, 16, 256, 9, 0, 1, None) == -2
    assert L.qmm_gemv_q8(_lib.QMM_Q4_K, dummy, _xq(16), dummy, 16, 256, 0, 0, 1, None) == -2
    # odd block count for the SoA layout
    assert L.qmm_gemv_q8(_lib.QMM_Q6_K_SOA, dummy, _xq(16), dummy, 16, 768, 1, 0, 1, None) == -2
    # null pointers
    assert L.qmm_gemv_q8(_lib.QMM_Q4_K, None, _xq(16), dummy, 16, 256, 1, 0, 1, None) == -3
    assert L.qmm_gemv_q8(_lib.QMM_Q4_K, dummy, _lib.XQ8(0, 0, 0, 0), dummy, 16, 256, 1, 0, 1, None) == -3
    # knobs: any tpr / rpt is accepted (as the reference's); the interleaved layouts' own limits
    assert L.qmm_gemv_q8(_lib.QMM_Q6_K_SOA, dummy, _xq(16), dummy, 16, 512, 1, 0, 5, None) == -1     # rpt 5: block formats
    assert L.qmm_gemv_q8(_lib.QMM_Q4_K, dummy, _xq(16), dummy, 12, 256, 1, 0, 5, None) == -2         # N % 8
    assert L.qmm_gemv_q8(_lib.QMM_Q4_K, dummy, _xq(16), dummy, 16, 256, 9, 0, 5, None) == -2         # 8 columns
    assert L.qmm_gemv_q8(_lib.QMM_Q5_1_SOA, dummy, _xq(16), dummy, 16, 512, 1, 3, 4, None) == -1     # 16-row layout
    assert L.qmm_gemv_q8(_lib.QMM_Q8_0_SOA, dummy, _xq(16), dummy, 16, 320, 1, 3, 4, None) == -2     # K % 256
    assert L.qmm_gemv_q8(_lib.QMM_Q4_K, dummy, _xq(16), dummy, 16, 256, 17, 3, 4, None) == -2        # 16 columns
    assert L.qmm_quantize_x_q8(None, _xq(16), 1, 256, None) == -3
    assert L.qmm_quantize_x_q8(dummy, _xq(16), 1, 100, None) == -2
    assert L.qmm_gemv_q4_K_f32(dummy, dummy, dummy, 16, 200, 1, 0, None) == -2
    seg = (_lib.GemvSeg * 2)(_lib.GemvSeg(0, 16, 16, 16, 256), _lib.GemvSeg(0, 16, 16, 16, 512))
    assert L.qmm_gemv_multi(seg, 2, _xq(16), 1, None) == -2          # K differs between segments
    assert L.qmm_gemv_multi(seg, 5, _xq(16), 1, None) == -2


def test_moe_argument_validation_without_device_work():
    L = _lib.lib()
    d = ctypes.c_void_p(16)
    assert L.qmm_moe_route(None, d, d, 1, None) == -3
    assert L.qmm_moe_route_n(d, d, d, 1, 512, 512, 10, None) == -2        # stride must hold the shared gate logit
    assert L.qmm_moe_route_n(d, d, d, 1, 2048, 2049, 10, None) == -2      # too many experts
    assert L.qmm_moe_route_n(d, d, d, 1, 64, 65, 17, None) == -2          # top-k above 16
    assert L.qmm_moe_route_n(d, d, d, 0, 64, 65, 4, None) == 0            # empty batch: nothing to do
    segs = _lib.MoeSegs()
    for g in range(2):
        segs.w[g] = 16; segs.shared[g] = 16; segs.y[g] = 16
    segs.ebytes = 1024
    assert L.qmm_gemv_moe(_lib.QMM_Q6_K, _lib.QMM_Q4_K, ctypes.byref(segs), 2, d, 11, _xq(16), 512, 2048, 1, 0, None) == -1
    assert L.qmm_gemv_moe(_lib.QMM_Q4_K, _lib.QMM_Q4_K, ctypes.byref(segs), 2, d, 11, _xq(16), 512, 2000, 1, 0, None) == -2
    assert L.qmm_gemv_moe(_lib.QMM_Q4_K, _lib.QMM_Q4_K, ctypes.byref(segs), 2, d, 17, _xq(16), 512, 2048, 1, 0, None) == -2
    assert L.qmm_gemv_moe(_lib.QMM_Q4_K, _lib.QMM_Q4_K, ctypes.byref(segs), 2, d, 11, _xq(16), 512, 2048, 65, 0, None) == -2
    assert L.qmm_gemv_moe(_lib.QMM_Q4_K, _lib.QMM_Q4_K, None, 2, d, 11, _xq(16), 512, 2048, 1, 0, None) == -3
    segs.slotw = 16
    assert L.qmm_gemv_moe(_lib.QMM_Q4_K, _lib.QMM_Q4_K, ctypes.byref(segs), 2, d, 11, _xq(16), 512, 2048, 1, 1, None) == -6
    # formats: the shared expert in the routed format or Q8_0_SOA; no Q6_K experts; K granules
    assert L.qmm_gemv_moe(_lib.QMM_Q5_1_SOA, _lib.QMM_Q5_K, ctypes.byref(segs), 1, d, 11, _xq(16), 512, 640, 1, 0, None) == -1
    assert L.qmm_gemv_moe(_lib.QMM_Q6_K_SOA, _lib.QMM_Q6_K_SOA, ctypes.byref(segs), 1, d, 11, _xq(16), 512, 512, 1, 0, None) == -1
    assert L.qmm_gemv_moe(_lib.QMM_Q5_1_SOA, _lib.QMM_Q8_0_SOA, ctypes.byref(segs), 1, d, 11, _xq(16), 512, 608, 1, 0, None) == -2
    assert L.qmm_gemv_moe(_lib.QMM_Q5_K, _lib.QMM_Q5_K, ctypes.byref(segs), 1, d, 11, _xq(16), 512, 640, 1, 0, None) == -2
    # no shared expert (NULL): accepted in the routed format (negative ids read expert 0), refused beside
    # a Q8_0_SOA shared format; T = 0 runs nothing
    segs.slotw = None
    segs.shared[0] = None
    assert L.qmm_gemv_moe(_lib.QMM_Q4_K, _lib.QMM_Q4_K, ctypes.byref(segs), 1, d, 11, _xq(16), 512, 2048, 0, 0, None) == 0
    assert L.qmm_gemv_moe(_lib.QMM_Q4_K, _lib.QMM_Q8_0_SOA, ctypes.byref(segs), 1, d, 11, _xq(16), 512, 2048, 0, 0, None) == -3
    assert L.qmm_moe_silu_quant(d, d, _xq(16), 4, 100, None) == -2
    assert L.qmm_moe_combine_sorted(d, d, None, d, 4, 11, 2048, None) == -3


def test_activation_producer_validation_without_device_work():
    L = _lib.lib()
    d = ctypes.c_void_p(16)
    assert L.qmm_add_rmsnorm_quant(d, None, d, d, _xq(16), 1, 5000, 1e-6, None) == -2      # n % 32 != 0
    assert L.qmm_add_rmsnorm_quant(d, None, d, d, _xq(16), 1, 16416, 1e-6, None) == -2     # n above 16384
    assert L.qmm_add_rmsnorm_quant(d, None, d, None, _xq(16), 1, 5120, 1e-6, None) == -3   # xn missing
    assert L.qmm_add_rmsnorm_quant(d, None, d, d, _lib.XQ8(16, 0, 16, 0), 1, 5120, 1e-6, None) == -3
    assert L.qmm_add_rmsnorm_quant(d, None, d, d, _xq(16), 0, 5120, 1e-6, None) == 0       # empty batch
    assert L.qmm_add_rmsnorm_quant(d, None, d, d, _xq(16), -1, 5120, 1e-6, None) == -2
    assert L.qmm_add_rmsnorm_bf16(d, None, d, None, 1, 5120, 1e-6, None) == -3
    assert L.qmm_add_rmsnorm_bf16(d, None, d, d, 1, 20000, 1e-6, None) == -2
    assert L.qmm_add_rmsnorm_bf16(d, None, d, d, 0, 77, 1e-6, None) == 0
    assert L.qmm_silu_mul_quant(d, d, _xq(16), 100, None) == -2
    assert L.qmm_silu_mul_quant(None, d, _xq(16), 128, None) == -3
    assert L.qmm_silu_mul_quant(d, d, _xq(16), 0, None) == 0
    assert L.qmm_silu_mul_bf16(d, None, d, 128, None) == -3
    assert L.qmm_silu_mul_bf16(d, d, d, 0, None) == 0


def test_router_validation_without_device_work():
    L = _lib.lib()
    d = ctypes.c_void_p(256)
    assert L.qmm_f32_gemv(d, d, d, 513, 2050, 1, None) == -2           # K % 4 != 0
    assert L.qmm_f32_gemv(d, ctypes.c_void_p(260), d, 513, 2048, 1, None) == -6   # x not 16-byte aligned
    assert L.qmm_f32_gemv(None, d, d, 513, 2048, 1, None) == -3
    assert L.qmm_f32_gemv(d, d, d, 0, 2048, 1, None) == 0
    assert L.qmm_gemm_f32(d, d, d, 2048, 513, 2562, None) == -2            # K % 4 != 0
    assert L.qmm_gemm_f32(ctypes.c_void_p(264), d, d, 2048, 513, 2560, None) == -6   # A not 16-byte aligned
    assert L.qmm_gemm_f32(d, d, None, 2048, 513, 2560, None) == -3
    assert L.qmm_gemm_f32(d, d, d, 0, 513, 2560, None) == 0                # nothing to do: no launch
    assert L.qmm_moe_router(d, d, d, d, d, 1, 2048, 2048, 10, None) == -2  # too many experts for the routing
    assert L.qmm_moe_router(d, d, d, d, d, 1, 512, 2048, 17, None) == -2   # top-k above 16
    assert L.qmm_moe_router(d, d, d, None, d, 1, 512, 2048, 10, None) == -3


def test_prefill_argument_validation_without_device_work():
    L = _lib.lib()
    d = ctypes.c_void_p(16)
    assert L.qmm_gemm_wq(_lib.QMM_Q6_K, d, d, d, 64, 64, 256, None) == -1        # GGUF Q6_K: dequant_bf16 + gemm_bf16
    assert L.qmm_gemm_wq(_lib.QMM_Q6_K_SOA, d, d, d, 64, 64, 768, None) == -2    # Q6_K_SOA: K % 512
    assert L.qmm_gemm_wq(_lib.QMM_Q5_1_SOA, d, d, d, 64, 64, 96, None) == -2     # SoA formats: K % 128
    assert L.qmm_gemm_wq(_lib.QMM_Q5_K, d, d, d, 64, 64, 384, None) == -2
    q4, q6 = _lib.QMM_Q4_K, _lib.QMM_Q6_K
    assert L.qmm_moe_sort(None, 4, 11, 512, 128, d, d, d, d, None) == -3
    assert L.qmm_moe_sort(d, 4, 11, 4096, 128, d, d, d, d, None) == -2       # more experts than the sort holds
    assert L.qmm_moe_sort(d, 4, 11, 512, 0, d, d, d, d, None) == -2
    args = (d, d, 1024, d, d, 8, d, d, d)
    assert L.qmm_moe_gemm_bf16(q6, q4, *args, 512, 2048, None) == -1
    assert L.qmm_moe_gemm_bf16(q4, q4, None, d, 1024, d, d, 8, d, d, d, 512, 2048, None) == -3
    assert L.qmm_moe_gemm_bf16(q4, q4, *args, 512, 2000, None) == -2
    assert L.qmm_moe_gemm_bf16(q4, q4, d, d, 1024, d, d, 0, d, d, d, 512, 2048, None) == 0   # no tiles: nothing to do
    gu = (d, d, d, d, 1024, d, d, 8, d, d, d)
    assert L.qmm_moe_gemm_gate_up_bf16(q4, q6, *gu, 512, 2048, None) == -1
    assert L.qmm_moe_gemm_gate_up_bf16(q4, q4, d, d, None, d, 1024, d, d, 8, d, d, d, 512, 2048, None) == -3
    assert L.qmm_moe_gemm_gate_up_bf16(q4, q4, *gu, 0, 2048, None) == -2
    assert L.qmm_gemm_wq(q6, d, d, d, 16, 16, 256, None) == -1
    assert L.qmm_gemm_wq(q4, d, d, d, 16, 16, 300, None) == -2
    assert L.qmm_gemm_wq(q4, d, None, d, 16, 16, 256, None) == -3
    assert L.qmm_gemm_bf16(d, d, d, 16, 16, 100, None) == -2
    assert L.qmm_dequant_bf16(q4, d, d, 16, 100, None) == -2
    assert L.qmm_dequant_bf16(99, d, d, 16, 256, None) == -1
    assert L.qmm_dequant_bf16(_lib.QMM_Q5_K, d, d, 16, 100, None) == -2
    assert L.qmm_gemv_q8_f32x(q6, d, d, d, 16, 256, 1, None) == -1
    assert L.qmm_gemv_q8_f32x(q4, d, None, d, 16, 256, 1, None) == -3
    assert L.qmm_gemv_q8_f32x(q4, d, d, d, 16, 256, 5, None) == -2      # ncol above 4
    assert L.qmm_gemv_q8_f32x(q4, d, d, d, 16, 6400, 1, None) == -2     # K above 6144


def test_off_path_entry_point_refused():
    """hc_up_fused (the reference's Flash-Next hyper-connection prologue, gemv.h:52) lies off the
    quantized matmul path: declared for the reference's callers, refused before any launch."""
    L = _lib.lib()
    buf = np.zeros(64, np.float32)
    assert L.qmm_hc_up_fused(buf.ctypes.data, buf.ctypes.data, 1, buf.ctypes.data, 32, 1, None) == -10
    assert "off the quantized matmul path" in L.qmm_status_string(-10).decode()
