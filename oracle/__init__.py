"""ctypes binding of the CPU oracle (oracle/liboracle.so), of the reference's own quant.h
(oracle/_ref/libqmm_ref.so) and of the reference's gemv.hip layout helpers
(oracle/_ref/libqmm_ref_gemv.so), the latter two when they were built.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker.  The product package (hipster_amd/) never imports it.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(_HERE, "liboracle.so")
REF_LIB = os.path.join(_HERE, "_ref", "libqmm_ref.so")
REF_GEMV_LIB = os.path.join(_HERE, "_ref", "libqmm_ref_gemv.so")
REF_GGUF_LIB = os.path.join(_HERE, "_ref", "libgguf_ref.so")

Q4_K, Q5_K, IQ4_XS, Q6_K_SOA, Q8_0_SOA, Q5_1_SOA, Q6_K = 0, 1, 2, 3, 4, 5, 6
Q8_0, Q5_1, Q5_0 = 8, 9, 10
_o = None
_r = None
_rg = None
_rgg = None

P = ctypes.c_void_p
I = ctypes.c_int


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def lib():
    global _o
    if _o is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} missing: run make -C oracle")
        L = ctypes.CDLL(LIB)
        L.qo_f16_to_f32.restype = ctypes.c_float
        L.qo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.qo_f32_to_bf16.restype = ctypes.c_uint16
        L.qo_f32_to_bf16.argtypes = [ctypes.c_float]
        L.qo_f32_to_f16.restype = ctypes.c_uint16
        L.qo_f32_to_f16.argtypes = [ctypes.c_float]
        L.qo_k_granule.restype = I
        L.qo_block_sum1024.restype = ctypes.c_float
        L.qo_block_sum1024.argtypes = [P]
        L.qo_k_granule.argtypes = [I]
        L.qo_row_bytes.restype = ctypes.c_size_t
        L.qo_row_bytes.argtypes = [I, I]
        for name, args in {
            "qo_scale_min_k4": [I, P, P, P],
            "qo_dequant_q4_K_block": [P, P], "qo_dequant_q6_K_block": [P, P],
            "qo_repack_row_q6_K": [P, P, I],
            "qo_dequant_q5_K_block": [P, P], "qo_dequant_iq4_xs_block": [P, P], "qo_dequant_q8_0_block": [P, P],
            "qo_dequant_q5_1_block": [P, P], "qo_dequant_q5_0_block": [P, P],
            "qo_repack_row_q8_0": [P, P, I], "qo_repack_row_q5_1": [P, P, I], "qo_repack_row_q5_0": [P, P, I],
            "qo_dequant_row": [I, P, P, I],
            "qo_dequant_matrix": [I, P, I, I, P, I], "qo_dequant_matrix_bf16": [I, P, I, I, P, I],
            "qo_quantize_x_q8": [P, I, P, P, P], "qo_q8_to_f32": [P, P, I, P],
            "qo_quantize_x_q8k": [P, I, I, P, P, P],
            "qo_silu_mul": [P, P, ctypes.c_size_t, P],
            "qo_add_rmsnorm_quant": [P, P, P, P, P, P, P, I, I, ctypes.c_float],
            "qo_add_rmsnorm_bf16": [P, P, P, P, I, I, ctypes.c_float],
            "qo_gemv_ref": [I, P, I, I, P, I, P, P, I],
            "qo_gemv_ref_rows": [I, P, I, I, P, I, P, I, P, P],
            "qo_gemv_f32": [I, P, I, I, P, I, P, I],
            "qo_moe_route": [P, I, I, I, I, P, P],
            "qo_f32_gemv": [P, P, P, I, I, I],
            "qo_moe_sort": [P, I, I, I, P, P, P, P],
            "qo_moe_decode": [I, P, P, P, ctypes.c_size_t, ctypes.c_size_t, P, P, P, P, P, P, I, I, I, I, P, P, P, P],
            "qo_moe_down_q8": [I, P, ctypes.c_size_t, P, P, P, P, P, I, I, I, I, P, P],
            "qo_moe_prefill_tokens": [I, P, P, P, ctypes.c_size_t, ctypes.c_size_t, P, P, P, P, P, P, I, I, I, P, I, P, I],
            "qo_gemm_wq_ref": [I, P, P, I, I, I, P, P, I, P],
        }.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = None if (name.startswith("qo_dequant_q") and name.endswith("_block")) or name.startswith("qo_repack_row") \
                or name in ("qo_scale_min_k4", "qo_quantize_x_q8", "qo_q8_to_f32", "qo_silu_mul", "qo_moe_route") else I
        _o = L
    return _o


def ref_lib():
    """The reference's quant.h compiled by oracle/Makefile, or None when it was not built."""
    global _r
    if _r is None and os.path.exists(REF_LIB):
        L = ctypes.CDLL(REF_LIB)
        L.ref_f16_to_f32.restype = ctypes.c_float
        L.ref_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.ref_get_scale_min_k4.argtypes = [I, P, P, P]
        L.ref_get_scale_min_k4.restype = None
        L.ref_dequant_row.argtypes = [I, P, P, ctypes.c_uint64]
        L.ref_dequant_row.restype = None
        L.ref_f32_to_f16.restype = ctypes.c_uint16
        L.ref_f32_to_f16.argtypes = [ctypes.c_float]
        L.ref_quantize_row_q8_0_soa.argtypes = [P, P, ctypes.c_uint64]
        L.ref_quantize_row_q8_0_soa.restype = None
        L.ref_gemv_f32_threads.argtypes = [I, P, ctypes.c_size_t, I, I, P, P, I]
        L.ref_gemv_f32_threads.restype = I
        _r = L
    return _r


# ---------------------------------------------------------------- numpy-facing helpers
def row_bytes(fmt, K):
    return lib().qo_row_bytes(fmt, K)


def dequant_rows(fmt, W, K, nthreads=8):
    """W uint8 [N][row_bytes] -> f32 [N][K]."""
    W = np.ascontiguousarray(W, dtype=np.uint8)
    N = W.shape[0]
    out = np.empty((N, K), dtype=np.float32)
    if lib().qo_dequant_matrix(fmt, _ptr(W), N, K, _ptr(out), nthreads) != 0:
        raise ValueError("dequant_matrix")
    return out


def dequant_rows_bf16(fmt, W, K, nthreads=8):
    W = np.ascontiguousarray(W, dtype=np.uint8)
    N = W.shape[0]
    out = np.empty((N, K), dtype=np.uint16)
    if lib().qo_dequant_matrix_bf16(fmt, _ptr(W), N, K, _ptr(out), nthreads) != 0:
        raise ValueError("dequant_matrix_bf16")
    return out


def quantize_x_q8(x):
    """x f32 [ncol][K] -> (q int8, d f32 [ncol][K/32], s f32)."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    ncol, K = x.shape
    q = np.empty((ncol, K), dtype=np.int8)
    d = np.empty((ncol, K // 32), dtype=np.float32)
    s = np.empty((ncol, K // 32), dtype=np.float32)
    for c in range(ncol):
        lib().qo_quantize_x_q8(_ptr(x[c]), K, _ptr(q[c]), _ptr(d[c]), _ptr(s[c]))
    return q, d, s


def quantize_x_q8k(x):
    """x f32 [ncol <= 16][K] -> (q int8 [ncol][K], d f32 [K/256][16], bs int16 [K/256][16][8]) (gemv.hip:686-705)."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    ncol, K = x.shape
    q = np.zeros((ncol, K), dtype=np.int8)
    d = np.zeros((K // 256, 16), dtype=np.float32)
    bs = np.zeros((K // 256, 16, 8), dtype=np.int16)
    lib().qo_quantize_x_q8k(_ptr(x), K, ncol, _ptr(q), _ptr(d), _ptr(bs))
    return q, d, bs


def q8k_to_f32(q, d):
    """The value each q8k entry stands for, q * (its 256-block's d), f32 [ncol][K]."""
    ncol, K = q.shape
    scale = np.repeat(d[:, :ncol].T, 256, axis=1)
    return (q.astype(np.float32) * scale).astype(np.float32)


def add_rmsnorm_quant(x, y, w, eps):
    """ops.hip:79-98 over rows of x [T][n]: returns (x + y, xn, q, d, s); x is not modified."""
    x = np.array(np.atleast_2d(x), dtype=np.float32, order="C", copy=True)
    T, n = x.shape
    yy = None if y is None else np.ascontiguousarray(np.atleast_2d(y), dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    xn = np.empty_like(x)
    q = np.empty((T, n), dtype=np.int8)
    d = np.empty((T, n // 32), dtype=np.float32)
    s = np.empty((T, n // 32), dtype=np.float32)
    if lib().qo_add_rmsnorm_quant(_ptr(x), None if yy is None else _ptr(yy), _ptr(w), _ptr(xn), _ptr(q), _ptr(d), _ptr(s),
                                  T, n, eps) != 0:
        raise ValueError("add_rmsnorm_quant: n")
    return x, xn, q, d, s


def add_rmsnorm_bf16(x, y, w, eps):
    """ops.hip:111-120 over rows of x [T][n]: returns (x + y, xb uint16 bits)."""
    x = np.array(np.atleast_2d(x), dtype=np.float32, order="C", copy=True)
    T, n = x.shape
    yy = None if y is None else np.ascontiguousarray(np.atleast_2d(y), dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    xb = np.empty((T, n), dtype=np.uint16)
    if lib().qo_add_rmsnorm_bf16(_ptr(x), None if yy is None else _ptr(yy), _ptr(w), _ptr(xb), T, n, eps) != 0:
        raise ValueError("add_rmsnorm_bf16: n")
    return x, xb


def block_sum1024(part):
    part = np.ascontiguousarray(part, dtype=np.float32)
    assert part.shape == (1024,)
    return lib().qo_block_sum1024(_ptr(part))


def q8_to_f32(q, d):
    q = np.ascontiguousarray(np.atleast_2d(q), dtype=np.int8)
    d = np.ascontiguousarray(np.atleast_2d(d), dtype=np.float32)
    ncol, K = q.shape
    out = np.empty((ncol, K), dtype=np.float32)
    for c in range(ncol):
        lib().qo_q8_to_f32(_ptr(q[c]), _ptr(d[c]), K, _ptr(out[c]))
    return out


def gemv_ref(fmt, W, N, K, x, nthreads=8):
    """double-precision y [ncol][N] and |w*x| sums (bench_gemv.cpp:95-104)."""
    W = np.ascontiguousarray(W, dtype=np.uint8)
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    ncol = x.shape[0]
    y = np.empty((ncol, N), dtype=np.float64)
    mag = np.empty((ncol, N), dtype=np.float64)
    if lib().qo_gemv_ref(fmt, _ptr(W), N, K, _ptr(x), ncol, _ptr(y), _ptr(mag), nthreads) != 0:
        raise ValueError("gemv_ref")
    return y, mag


def gemv_ref_rows(fmt, W, N, K, x, rows):
    W = np.ascontiguousarray(W, dtype=np.uint8)
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    ncol = x.shape[0]
    y = np.empty((ncol, len(rows)), dtype=np.float64)
    mag = np.empty((ncol, len(rows)), dtype=np.float64)
    if lib().qo_gemv_ref_rows(fmt, _ptr(W), N, K, _ptr(x), ncol, _ptr(rows), len(rows), _ptr(y), _ptr(mag)) != 0:
        raise ValueError("gemv_ref_rows")
    return y, mag


def gemv_f32(fmt, W, N, K, x, nthreads=1):
    """CPU baseline: dequant per row + fp32 dot, nthreads host threads."""
    W = np.ascontiguousarray(W, dtype=np.uint8)
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    y = np.empty((x.shape[0], N), dtype=np.float32)
    if lib().qo_gemv_f32(fmt, _ptr(W), N, K, _ptr(x), x.shape[0], _ptr(y), nthreads) != 0:
        raise ValueError("gemv_f32")
    return y


def ref_gemv_f32(gtype, W, N, K, x, nthreads=1):
    """The CPU baseline on the reference's own code (ref_shim.cpp: quant.h dequant_row + a sequential
    f32 dot per row, rows over nthreads threads); gtype is the GGUF type id (12 = Q4_K).  None when
    oracle/_ref was not built."""
    L = ref_lib()
    if L is None:
        return None
    W = np.ascontiguousarray(W, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    y = np.empty(N, dtype=np.float32)
    L.ref_gemv_f32_threads(gtype, _ptr(W), W.nbytes // N, N, K, _ptr(x), _ptr(y), nthreads)
    return y


def moe_route(logits, nexp=512, topk=10):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, stride = logits.shape
    ids = np.empty((T, topk + 1), dtype=np.int32)
    w = np.empty((T, topk + 1), dtype=np.float32)
    lib().qo_moe_route(_ptr(logits), T, nexp, stride, topk, _ptr(ids), _ptr(w))
    return ids, w


def f32_gemv(W, x):
    """fn.hip:251-277: W [N][K] f32, x [T][K] f32 -> y [T][N] (the reference's arithmetic and order)."""
    W = np.ascontiguousarray(W, dtype=np.float32)
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    N, K = W.shape
    T = x.shape[0]
    y = np.empty((T, N), dtype=np.float32)
    if lib().qo_f32_gemv(_ptr(W), _ptr(x), _ptr(y), N, K, T) != 0:
        raise ValueError("f32_gemv: K % 4 != 0")
    return y


def moe_sort(ids, maxc):
    """ids [T][NE] -> (kpos [T*NE], rowtok [T*NE], tiles [nt][3], stiles [nst][3])."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, NE = ids.shape
    NS = T * NE
    kpos = np.empty(NS, dtype=np.int32)
    rowtok = np.empty(NS, dtype=np.int32)
    tiles = np.empty((NS + 1, 3), dtype=np.int32)
    nst = ctypes.c_int(0)
    nt = lib().qo_moe_sort(_ptr(ids), T, NE, maxc, _ptr(kpos), _ptr(rowtok), _ptr(tiles), ctypes.byref(nst))
    return kpos, rowtok, tiles[:nt].copy(), tiles[nt:nt + nst.value].copy()


def moe_decode(fmt, Wg, Wu, Wd, Sg, Su, Sd, x, ids, w, H, F):
    """Per-token decode MoE (q8 activations): returns g, u [T*NE][F], dn [T*NE][H], y [T][H]."""
    Wg, Wu, Wd, Sg, Su, Sd = (np.ascontiguousarray(a, dtype=np.uint8) for a in (Wg, Wu, Wd, Sg, Su, Sd))
    x = np.ascontiguousarray(x, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    T, NE = ids.shape
    eb_gu, eb_d = Wg[0].nbytes, Wd[0].nbytes
    g = np.empty((T * NE, F), dtype=np.float32)
    u = np.empty((T * NE, F), dtype=np.float32)
    dn = np.empty((T * NE, H), dtype=np.float32)
    y = np.empty((T, H), dtype=np.float32)
    rc = lib().qo_moe_decode(fmt, _ptr(Wg), _ptr(Wu), _ptr(Wd), eb_gu, eb_d, _ptr(Sg), _ptr(Su), _ptr(Sd), _ptr(x),
                             _ptr(ids), _ptr(w), T, NE, H, F, _ptr(g), _ptr(u), _ptr(dn), _ptr(y))
    if rc != 0:
        raise ValueError("moe_decode")
    return g, u, dn, y


def moe_down_q8(fmt, Wd, Sd, hq, hd, ids, w, H, F):
    Wd, Sd = (np.ascontiguousarray(a, dtype=np.uint8) for a in (Wd, Sd))
    hq = np.ascontiguousarray(hq, dtype=np.int8)
    hd = np.ascontiguousarray(hd, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    T, NE = ids.shape
    dn = np.empty((T * NE, H), dtype=np.float32)
    y = np.empty((T, H), dtype=np.float32)
    rc = lib().qo_moe_down_q8(fmt, _ptr(Wd), Wd[0].nbytes, _ptr(Sd), _ptr(hq), _ptr(hd), _ptr(ids), _ptr(w), T, NE, H, F,
                              _ptr(dn), _ptr(y))
    if rc != 0:
        raise ValueError("moe_down_q8")
    return dn, y


def moe_prefill_tokens(fmt, Wg, Wu, Wd, Sg, Su, Sd, xb, ids, w, H, F, toks, nthreads=8):
    Wg, Wu, Wd, Sg, Su, Sd = (np.ascontiguousarray(a, dtype=np.uint8) for a in (Wg, Wu, Wd, Sg, Su, Sd))
    xb = np.ascontiguousarray(xb, dtype=np.uint16)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    toks = np.ascontiguousarray(toks, dtype=np.int32)
    NE = ids.shape[1]
    y = np.empty((len(toks), H), dtype=np.float32)
    rc = lib().qo_moe_prefill_tokens(fmt, _ptr(Wg), _ptr(Wu), _ptr(Wd), Wg[0].nbytes, Wd[0].nbytes, _ptr(Sg), _ptr(Su),
                                     _ptr(Sd), _ptr(xb), _ptr(ids), _ptr(w), NE, H, F, _ptr(toks), len(toks), _ptr(y),
                                     nthreads)
    if rc != 0:
        raise ValueError("moe_prefill_tokens")
    return y


def gemm_wq_ref(fmt, W, A_bf16, M, N, K, ms, ns):
    W = np.ascontiguousarray(W, dtype=np.uint8)
    A = np.ascontiguousarray(A_bf16, dtype=np.uint16)
    ms = np.ascontiguousarray(ms, dtype=np.int32)
    ns = np.ascontiguousarray(ns, dtype=np.int32)
    out = np.empty(len(ms), dtype=np.float64)
    if lib().qo_gemm_wq_ref(fmt, _ptr(W), _ptr(A), M, N, K, _ptr(ms), _ptr(ns), len(ms), _ptr(out)) != 0:
        raise ValueError("gemm_wq_ref")
    return out


def ref_gemv_lib():
    """The reference's engine/kernels/gemv.hip host layout helpers (row bytes, load-time repacks)
    compiled by oracle/Makefile, or None when they were not built.  Host functions only."""
    global _rg
    if _rg is None and os.path.exists(REF_GEMV_LIB):
        L = ctypes.CDLL(REF_GEMV_LIB)
        L.refg_wfmt_row_bytes.restype = ctypes.c_size_t
        L.refg_wfmt_row_bytes.argtypes = [I, I]
        for n in ("refg_repack_row_q6_K", "refg_repack_row_q8_0", "refg_repack_row_q5_1", "refg_repack_row_q5_0"):
            getattr(L, n).argtypes = [P, P, I]
            getattr(L, n).restype = None
        for n in ("refg_repack_interleave8", "refg_repack_wmma_il"):
            getattr(L, n).argtypes = [I, P, P, I, I]
            getattr(L, n).restype = None
        L.refg_wmma_il_bytes.restype = ctypes.c_size_t
        L.refg_wmma_il_bytes.argtypes = [I, I, I]
        _rg = L
    return _rg


def ref_gguf_lib():
    """The reference's GGUF v3 reader (engine/src/gguf.cpp) compiled by oracle/Makefile, or None when it
    was not built (no reference checkout)."""
    global _rgg
    if _rgg is None and os.path.exists(REF_GGUF_LIB):
        L = ctypes.CDLL(REF_GGUF_LIB)
        L.refgg_open.restype = P
        L.refgg_open.argtypes = [ctypes.c_char_p]
        L.refgg_close.argtypes = [P]
        L.refgg_close.restype = None
        L.refgg_n_tensors.restype = ctypes.c_long
        L.refgg_n_tensors.argtypes = [P]
        L.refgg_tensor.argtypes = [P, ctypes.c_long, ctypes.c_char_p, I, P, P, P, P, P]
        L.refgg_read.argtypes = [P, ctypes.c_char_p, P]
        L.refgg_kv_u32.argtypes = [P, ctypes.c_char_p, P]
        L.refgg_kv_f32.argtypes = [P, ctypes.c_char_p, P]
        L.refgg_kv_str.argtypes = [P, ctypes.c_char_p, ctypes.c_char_p, I]
        _rgg = L
    return _rgg
