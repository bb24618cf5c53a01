"""ctypes binding of libhipster_qmm.so (the C ABI declared in include/hipster_qmm.h).

The library is built in-tree by ``hipster_amd/csrc/Makefile`` (``__graft_entry__.build()``).  There
is no fallback: if the shared library is missing or fails to load, every call raises.
"""
import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libhipster_qmm.so")

# status codes and formats (include/hipster_qmm.h)
QMM_OK = 0
STATUS = {0: "QMM_OK", -1: "QMM_ERR_FORMAT", -2: "QMM_ERR_SHAPE", -3: "QMM_ERR_NULL",
          -4: "QMM_ERR_LAUNCH", -5: "QMM_ERR_WORKSPACE", -6: "QMM_ERR_ARG", -7: "QMM_ERR_LAYOUT", -8: "QMM_ERR_IO",
          -9: "QMM_ERR_NOT_FOUND", -10: "QMM_ERR_UNSUPPORTED"}
QMM_Q4_K, QMM_Q5_K, QMM_IQ4_XS, QMM_Q6_K_SOA, QMM_Q8_0_SOA, QMM_Q5_1_SOA, QMM_Q6_K = 0, 1, 2, 3, 4, 5, 6

c_vp = ctypes.c_void_p
c_int = ctypes.c_int


class XQ8(ctypes.Structure):
    """qmm_xq8 / reference XQ8 (engine/kernels/gemv.h:8)."""
    _fields_ = [("q", c_vp), ("d", c_vp), ("s", c_vp), ("ds", c_vp)]


class XQ8K(ctypes.Structure):
    """qmm_xq8k / reference XQ8K (engine/kernels/gemv.h:33)."""
    _fields_ = [("q", c_vp), ("d", c_vp), ("bs", c_vp)]


class GgufTensor(ctypes.Structure):
    """qmm_gguf_tensor / reference GTensor (engine/src/gguf.h:26-35)."""
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_int32), ("n_dims", ctypes.c_uint32), ("ne", ctypes.c_uint64 * 4),
                ("nbytes", ctypes.c_size_t), ("data", c_vp), ("shard", ctypes.c_int32), ("file_off", ctypes.c_uint64)]


class GemvSeg(ctypes.Structure):
    """qmm_gemv_seg / reference GemvSeg (engine/kernels/gemv.h:27)."""
    _fields_ = [("fmt", ctypes.c_int32), ("w", c_vp), ("y", c_vp), ("N", ctypes.c_int32), ("K", ctypes.c_int32)]


class MoeSegs(ctypes.Structure):
    """qmm_moe_segs / reference MoeSegs (engine/kernels/gemv.h:43)."""
    _fields_ = [("w", c_vp * 2), ("shared", c_vp * 2), ("y", c_vp * 2), ("ebytes", ctypes.c_size_t), ("slotw", c_vp)]


class MoeTile(ctypes.Structure):
    """qmm_moe_tile / reference MoeTile (engine/kernels/gemv.h:48)."""
    _fields_ = [("expert", ctypes.c_int32), ("k0", ctypes.c_int32), ("ncols", ctypes.c_int32)]


# name -> (restype, argtypes); every symbol the header declares
SIGNATURES = {
    "qmm_version": (ctypes.c_char_p, []),
    "qmm_status_string": (ctypes.c_char_p, [c_int]),
    "qmm_wfmt_row_bytes": (ctypes.c_size_t, [c_int, c_int]),
    "qmm_gtype_block": (c_int, [c_int, c_vp, c_vp]),
    "qmm_gguf_open": (c_int, [ctypes.c_char_p, ctypes.POINTER(c_vp)]),
    "qmm_gguf_close": (None, [c_vp]),
    "qmm_gguf_n_tensors": (ctypes.c_int64, [c_vp]),
    "qmm_gguf_mapped_bytes": (ctypes.c_size_t, [c_vp]),
    "qmm_gguf_tensor_at": (c_int, [c_vp, ctypes.c_int64, ctypes.POINTER(GgufTensor)]),
    "qmm_gguf_find": (c_int, [c_vp, ctypes.c_char_p, ctypes.POINTER(GgufTensor)]),
    "qmm_gguf_kv_kind": (c_int, [c_vp, ctypes.c_char_p, ctypes.POINTER(c_int)]),
    "qmm_gguf_kv_u32": (c_int, [c_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32)]),
    "qmm_gguf_kv_f32": (c_int, [c_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float)]),
    "qmm_gguf_kv_str": (c_int, [c_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p)]),
    "qmm_gguf_kv_array_len": (c_int, [c_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64)]),
    "qmm_gguf_read_tensor": (c_int, [c_vp, ctypes.c_char_p, c_vp, ctypes.c_size_t]),
    "qmm_weight_format": (c_int, [c_int, c_int, ctypes.POINTER(c_int), ctypes.POINTER(ctypes.c_size_t)]),
    "qmm_prepare_weight": (c_int, [c_int, c_vp, c_int, c_int, c_vp, c_int]),
    "qmm_repack_row_q6_K": (c_int, [c_vp, c_vp, c_int]),
    "qmm_repack_row_q8_0": (c_int, [c_vp, c_vp, c_int]),
    "qmm_repack_row_q5_1": (c_int, [c_vp, c_vp, c_int]),
    "qmm_repack_row_q5_0": (c_int, [c_vp, c_vp, c_int]),
    "qmm_repack_interleave8": (c_int, [c_int, c_vp, c_vp, c_int, c_int]),
    "qmm_wmma_il_bytes": (ctypes.c_size_t, [c_int, c_int, c_int]),
    "qmm_repack_wmma_il": (c_int, [c_int, c_vp, c_vp, c_int, c_int]),
    "qmm_quantize_x_q8": (c_int, [c_vp, XQ8, c_int, c_int, c_vp]),
    "qmm_gemv_q8": (c_int, [c_int, c_vp, XQ8, c_vp, c_int, c_int, c_int, c_int, c_int, c_vp]),
    "qmm_gemv_multi": (c_int, [ctypes.POINTER(GemvSeg), c_int, XQ8, c_int, c_vp]),
    "qmm_gemv_q8_f32x": (c_int, [c_int, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    "qmm_gemv_q4_K_f32": (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_vp]),
    "qmm_gemv_splitk": (c_int, [c_int, c_vp, XQ8, c_vp, c_int, c_int, c_int, c_int, c_vp]),
    "qmm_hc_up_fused": (c_int, [c_vp, c_vp, c_int, c_vp, c_int, c_int, c_vp]),
    "qmm_quantize_x_q8k": (c_int, [c_vp, XQ8K, c_int, c_int, c_vp]),
    "qmm_gemv_q8k": (c_int, [ctypes.POINTER(GemvSeg), c_int, XQ8K, c_int, c_vp]),
    "qmm_set_gemv_mfma_min_ncol": (c_int, [c_int]),
    "qmm_set_gemv_q6k_mfma_min_ncol": (c_int, [c_int]),
    "qmm_set_gemv_q80_mfma_min_ncol": (c_int, [c_int]),
    "qmm_set_gemv_fmt_xlds": (c_int, [c_int]),
    "qmm_moe_route": (c_int, [c_vp, c_vp, c_vp, c_int, c_vp]),
    "qmm_moe_route_n": (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_vp]),
    "qmm_gemv_moe": (c_int, [c_int, c_int, ctypes.POINTER(MoeSegs), c_int, c_vp, c_int, XQ8, c_int, c_int, c_int, c_int, c_vp]),
    "qmm_moe_silu_quant": (c_int, [c_vp, c_vp, XQ8, c_int, c_int, c_vp]),
    "qmm_moe_decode": (c_int, [c_int, c_vp, c_vp, c_vp, ctypes.c_size_t, ctypes.c_size_t, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int,
                               XQ8, c_int, c_int, c_int, c_vp, c_vp, c_vp, ctypes.c_size_t, c_vp, c_vp]),
    "qmm_moe_decode_ws_bytes": (ctypes.c_size_t, [c_int, c_int, c_int]),
    "qmm_moe_decode_noalloc": (c_int, [c_int, c_vp, c_vp, c_vp, ctypes.c_size_t, ctypes.c_size_t, c_vp, c_vp, c_vp, c_vp, c_int, c_int,
                                       c_int, XQ8, c_int, c_int, c_int, c_vp, c_vp, c_vp, c_vp]),
    "qmm_moe_decode_scratch_max": (ctypes.c_size_t, []),
    "qmm_moe_combine_sorted": (c_int, [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    "qmm_dequant_bf16": (c_int, [c_int, c_vp, c_vp, c_int, c_int, c_vp]),
    "qmm_moe_sort": (c_int, [c_vp, c_int, c_int, c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_vp]),
    "qmm_moe_gemm_bf16": (c_int, [c_int, c_int, c_vp, c_vp, ctypes.c_size_t, c_vp, c_vp, c_int, c_vp, c_vp, c_vp, c_int, c_int, c_vp]),
    "qmm_moe_gemm_gate_up_bf16": (c_int, [c_int, c_int, c_vp, c_vp, c_vp, c_vp, ctypes.c_size_t, c_vp, c_vp, c_int, c_vp, c_vp,
                                          c_vp, c_int, c_int, c_vp]),
    "qmm_moe_silu_bf16": (c_int, [c_vp, c_vp, c_vp, ctypes.c_size_t, c_vp]),
    "qmm_moe_gemm_q8": (c_int, [c_int, c_int, c_vp, c_vp, ctypes.c_size_t, c_vp, c_int, c_vp, c_int, c_int, c_vp, XQ8, c_vp,
                                c_int, c_int, c_vp]),
    "qmm_f32_gemv": (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    "qmm_gemm_f32": (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    "qmm_moe_router": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_vp]),
    "qmm_add_rmsnorm_quant": (c_int, [c_vp, c_vp, c_vp, c_vp, XQ8, c_int, c_int, ctypes.c_float, c_vp]),
    "qmm_add_rmsnorm_bf16": (c_int, [c_vp, c_vp, c_vp, c_vp, c_int, c_int, ctypes.c_float, c_vp]),
    "qmm_silu_mul_quant": (c_int, [c_vp, c_vp, XQ8, c_int, c_vp]),
    "qmm_silu_mul_bf16": (c_int, [c_vp, c_vp, c_vp, ctypes.c_size_t, c_vp]),
    "qmm_gemm_wq": (c_int, [c_int, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    "qmm_gemm_bf16": (c_int, [c_vp, c_vp, c_vp, c_int, c_int, c_int, c_vp]),
    "qmm_gemm_bf16_ld": (c_int, [c_vp, c_int, c_vp, c_int, c_vp, c_int, c_int, c_int, c_vp]),
    "qmm_f32_to_bf16": (c_int, [c_vp, c_vp, ctypes.c_size_t, c_vp]),
    "qmm_bf16_to_f32": (c_int, [c_vp, c_vp, ctypes.c_size_t, c_vp]),
    "qmm_bf16_to_f32_seg": (c_int, [c_vp, c_int, c_int, c_int, c_vp, c_int, c_vp]),
    "qmm_bf16_to_f32_seg2": (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_vp, c_int, c_vp]),
}

_lib = None


class QmmError(RuntimeError):
    pass


def lib():
    """Load libhipster_qmm.so once; raise if it is missing (no fallback path exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise QmmError(f"{LIB_PATH} not built: run __graft_entry__.build() (make -C hipster_amd/csrc)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name, None)
            if fn is None:
                continue  # reported by exported_symbols(); calling it raises AttributeError below
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    """Names from SIGNATURES that the loaded library actually exports."""
    L = lib()
    return [n for n in SIGNATURES if hasattr(L, n)]


def check(status, what=""):
    if status != QMM_OK:
        raise QmmError(f"{what}: {STATUS.get(status, status)}")
    return status
