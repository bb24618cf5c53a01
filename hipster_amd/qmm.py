"""Python mirror of the reference's hot-path call surface (``namespace hip`` in
engine/kernels/gemv.h, gemm.h and fn.h), over the C ABI of libhipster_qmm.so.

Same function names, argument meaning and output layout as the reference; torch CUDA tensors stand
in for the device pointers (torch is only the device-memory and stream plumbing here).  Errors that
the reference turns into ``abort()`` raise ``QmmError`` instead.  Every call launches on the current
torch stream unless ``stream`` is given.
"""
import ctypes

import torch

from . import _lib
from ._lib import GemvSeg, MoeSegs, MoeTile, QmmError, XQ8, XQ8K, check  # noqa: F401

WFmt = type("WFmt", (), {"Q4_K": _lib.QMM_Q4_K, "Q5_K": _lib.QMM_Q5_K, "IQ4_XS": _lib.QMM_IQ4_XS,
                         "Q6_K_SOA": _lib.QMM_Q6_K_SOA, "Q8_0_SOA": _lib.QMM_Q8_0_SOA,
                         "Q5_1_SOA": _lib.QMM_Q5_1_SOA, "Q6_K": _lib.QMM_Q6_K})


def _p(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _stream(stream):
    s = torch.cuda.current_stream() if stream is None else stream
    return ctypes.c_void_p(s.cuda_stream)


def _dev(t, dtype=None, name="tensor"):
    if t is None or not t.is_cuda:
        raise QmmError(f"{name} must be a CUDA tensor")
    if dtype is not None and t.dtype != dtype:
        raise QmmError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise QmmError(f"{name} must be contiguous")
    return t


class XQ8Buf:
    """Device buffers of XQ8 (gemv.h:8): q [ncol][K] int8, d/s [ncol][K/32] f32, optional ds."""

    def __init__(self, ncol, K, device="cuda", with_ds=False):
        self.ncol, self.K = ncol, K
        self.q = torch.zeros((ncol, K), dtype=torch.int8, device=device)
        self.d = torch.zeros((ncol, K // 32), dtype=torch.float32, device=device)
        self.s = torch.zeros((ncol, K // 32), dtype=torch.float32, device=device)
        self.ds = torch.zeros((ncol, K // 32, 2), dtype=torch.float32, device=device) if with_ds else None

    def c(self):
        return XQ8(self.q.data_ptr(), self.d.data_ptr(), self.s.data_ptr(), 0 if self.ds is None else self.ds.data_ptr())


class XQ8KBuf:
    """Device buffers of XQ8K (gemv.h:33): q [ncol][K] int8, d [K/256][16] f32, bs [K/256][16][8] int16."""

    def __init__(self, ncol, K, device="cuda"):
        self.ncol, self.K = ncol, K
        self.q = torch.zeros((ncol, K), dtype=torch.int8, device=device)
        self.d = torch.zeros((K // 256, 16), dtype=torch.float32, device=device)
        self.bs = torch.zeros((K // 256, 16, 8), dtype=torch.int16, device=device)

    def c(self):
        return XQ8K(self.q.data_ptr(), self.d.data_ptr(), self.bs.data_ptr())


def wfmt_row_bytes(fmt, K):
    return _lib.lib().qmm_wfmt_row_bytes(fmt, K)


def repack_row_q6_K(src, K):
    """Host repack of one GGUF Q6_K row (bytes) to the SoA layout (gemv.hip:1341-1350)."""
    import numpy as np
    src = np.ascontiguousarray(src, dtype=np.uint8)
    dst = np.empty_like(src)
    check(_lib.lib().qmm_repack_row_q6_K(src.ctypes.data, dst.ctypes.data, K), "repack_row_q6_K")
    return dst


def _repack(name, src, K, dst_bytes):
    import numpy as np
    src = np.ascontiguousarray(src, dtype=np.uint8)
    dst = np.empty(dst_bytes, dtype=np.uint8)
    check(getattr(_lib.lib(), "qmm_" + name)(src.ctypes.data, dst.ctypes.data, K), name)
    return dst


def repack_row_q8_0(src, K):
    """Host repack of one GGUF Q8_0 row to the Q8_0_SOA layout (gemv.h:16, gemv.hip:1351-1354)."""
    return _repack("repack_row_q8_0", src, K, K + K // 16)


def repack_row_q5_1(src, K):
    """Host repack of one GGUF Q5_1 row to the Q5_1_SOA layout (gemv.h:17, gemv.hip:1458-1465)."""
    return _repack("repack_row_q5_1", src, K, K // 32 * 24)


def repack_row_q5_0(src, K):
    """Host repack of one GGUF Q5_0 row to the Q5_1_SOA layout, m = -16 d (gemv.h:18, gemv.hip:1448-1457)."""
    return _repack("repack_row_q5_0", src, K, K // 32 * 24)


def repack_interleave8(fmt, src, N, K):
    """Host 8-row block interleave of a whole matrix (gemv.h:21, gemv.hip:1442-1447)."""
    import numpy as np
    src = np.ascontiguousarray(src, dtype=np.uint8)
    dst = np.empty_like(src)
    check(_lib.lib().qmm_repack_interleave8(fmt, src.ctypes.data, dst.ctypes.data, N, K), "repack_interleave8")
    return dst


def wmma_il_bytes(fmt, N, K):
    return _lib.lib().qmm_wmma_il_bytes(fmt, N, K)


def repack_wmma_il(fmt, src, N, K):
    """Host 16-row piece-major layout of a whole matrix (gemv.h:37-38, gemv.hip:1280-1303)."""
    import numpy as np
    src = np.ascontiguousarray(src, dtype=np.uint8)
    dst = np.empty(wmma_il_bytes(fmt, N, K), dtype=np.uint8)
    check(_lib.lib().qmm_repack_wmma_il(fmt, src.ctypes.data, dst.ctypes.data, N, K), "repack_wmma_il")
    return dst


def quantize_x_q8(x, out, ncol, K, stream=None):
    """gemv.h:10: x f32 [ncol][K] -> out (XQ8Buf)."""
    _dev(x, torch.float32, "x")
    check(_lib.lib().qmm_quantize_x_q8(_p(x), out.c(), ncol, K, _stream(stream)), "quantize_x_q8")


def gemv_q8(fmt, W, x, y, N, K, ncol, tpr=0, rpt=1, stream=None):
    """gemv.h:25: y[c][n] = W[n] . x[c] for c < ncol (x an XQ8Buf)."""
    _dev(W, torch.uint8, "W"); _dev(y, torch.float32, "y")
    check(_lib.lib().qmm_gemv_q8(fmt, _p(W), x.c(), _p(y), N, K, ncol, tpr, rpt, _stream(stream)), "gemv_q8")


def _segs(segs):
    arr = (GemvSeg * len(segs))()
    for i, (fmt, w, y, N, K) in enumerate(segs):
        arr[i] = GemvSeg(fmt, w.data_ptr(), y.data_ptr(), N, K)
    return arr


def gemv_multi(segs, x, ncol, stream=None):
    """gemv.h:28: segs = [(fmt, W, y, N, K), ...] sharing x."""
    arr = _segs(segs)
    check(_lib.lib().qmm_gemv_multi(arr, len(segs), x.c(), ncol, _stream(stream)), "gemv_multi")


def gemv_wmma_ok(segs):
    """gemv.h:35: the library's GEMV is T-invariant for every supported format, so any segment list
    of Q4_K / Q6_K_SOA weights with K % 256 == 0 qualifies."""
    return 1 <= len(segs) <= 4 and all(f in (WFmt.Q4_K, WFmt.Q6_K_SOA) and K % 256 == 0 for f, _, _, _, K in segs)


def gemv_wmma(segs, x, ncol, mode=0, stream=None):
    """gemv.h:36: the reference's T-invariant matrix-core GEMV; here the (T-invariant) multi GEMV,
    mode accepted and ignored."""
    gemv_multi(segs, x, ncol, stream)


def gemv_splitk(fmt, W, x, part, N, K, ksplit, ncol, stream=None):
    """gemv.h:55: part[(c*ksplit + ks)][N] = W . x over the ks-th range of 256-weight blocks."""
    _dev(W, torch.uint8, "W"); _dev(part, torch.float32, "part")
    check(_lib.lib().qmm_gemv_splitk(fmt, _p(W), x.c(), _p(part), N, K, ksplit, ncol, _stream(stream)), "gemv_splitk")


def quantize_x_q8k(x, out, ncol, K, stream=None):
    """gemv.h:34: x f32 [ncol][K] -> out (XQ8KBuf): one scale per 256, int16 sums per 32."""
    _dev(x, torch.float32, "x")
    check(_lib.lib().qmm_quantize_x_q8k(_p(x), out.c(), ncol, K, _stream(stream)), "quantize_x_q8k")


def gemv_wmma_q8k(segs, x, ncol, ks_mode=0, stream=None):
    """gemv.h:35: segs = [(fmt, W, y, N, K), ...] on Q8_K activations (x an XQ8KBuf); ks_mode accepted."""
    arr = _segs(segs)
    check(_lib.lib().qmm_gemv_q8k(arr, len(segs), x.c(), ncol, _stream(stream)), "gemv_wmma_q8k")


def gemv_q8_f32x(fmt, W, x, y, N, K, ncol, stream=None):
    """quantize_x_q8 + gemv_q8 in one launch (f32 x in), bit for bit the same y."""
    check(_lib.lib().qmm_gemv_q8_f32x(fmt, _p(W), _p(x), _p(y), N, K, ncol, _stream(stream)), "gemv_q8_f32x")


def gemv_q4_K_f32(W, x, y, N, K, ncol, tpr=0, stream=None):
    """gemv.h:57: f32-activation Q4_K GEMV."""
    _dev(W, torch.uint8, "W"); _dev(x, torch.float32, "x"); _dev(y, torch.float32, "y")
    check(_lib.lib().qmm_gemv_q4_K_f32(_p(W), _p(x), _p(y), N, K, ncol, tpr, _stream(stream)), "gemv_q4_K_f32")


def moe_route(logits, ids, w, T, stream=None):
    """fn.h:43: logits [T][513] -> ids/w [T][11] (10 routed + shared)."""
    check(_lib.lib().qmm_moe_route(_p(logits), _p(ids), _p(w), T, _stream(stream)), "moe_route")


def moe_route_n(logits, ids, w, T, nexp, stride, topk, stream=None):
    check(_lib.lib().qmm_moe_route_n(_p(logits), _p(ids), _p(w), T, nexp, stride, topk, _stream(stream)), "moe_route_n")


def gemv_moe(fmt, shared_fmt, w, shared, y, ebytes, ids, nexp, x, N, K, T, xrow_te, slotw=None, stream=None):
    """gemv.h:44: w/shared/y are lists of 1 or 2 tensors (gate|up share a launch)."""
    nseg = len(w)
    a = MoeSegs()
    for g in range(nseg):
        a.w[g] = w[g].data_ptr(); a.shared[g] = shared[g].data_ptr(); a.y[g] = y[g].data_ptr()
    a.ebytes = ebytes
    a.slotw = 0 if slotw is None else slotw.data_ptr()
    check(_lib.lib().qmm_gemv_moe(fmt, shared_fmt, ctypes.byref(a), nseg, _p(ids), nexp, x.c(), N, K, T, int(xrow_te),
                                  _stream(stream)), "gemv_moe")


def moe_decode_ws_bytes(T, topk, F):
    return _lib.lib().qmm_moe_decode_ws_bytes(T, topk, F)


def moe_decode(fmt, Wg, Wu, Wd, ebytes_gu, ebytes_d, Sg, Su, Sd, logits, stride, nexp_total, topk, x, T, H, F, ids, w, ws, y,
               stream=None):
    """The MoE decode step in one call (T = 1: two launches, routing + gate|up + silu * up -> q8, then the
    down projection; T > 1: the four launches); ids / w [T][topk+1] and y [T][H] out, bitwise moe_route + gemv_moe +
    moe_silu_quant + gemv_moe.  ws: a device buffer of moe_decode_ws_bytes(T, topk, F) bytes."""
    check(_lib.lib().qmm_moe_decode(fmt, _p(Wg), _p(Wu), _p(Wd), ebytes_gu, ebytes_d, _p(Sg), _p(Su), _p(Sd), _p(logits), stride,
                                    nexp_total, topk, x.c(), T, H, F, _p(ids), _p(w), _p(ws), ws.numel() * ws.element_size(),
                                    _p(y), _stream(stream)), "moe_decode")


def moe_decode_noalloc(fmt, Wg, Wu, Wd, ebytes_gu, ebytes_d, Sg, Su, Sd, logits, stride, nexp_total, topk, x, T, H, F, ids, w, y,
                       stream=None):
    """moe_decode with its workspace in the library's static per-GPU array (no allocation; calls that
    overlap on one GPU race); QmmError(-5) when moe_decode_ws_bytes(T, topk, F) > moe_decode_scratch_max()."""
    check(_lib.lib().qmm_moe_decode_noalloc(fmt, _p(Wg), _p(Wu), _p(Wd), ebytes_gu, ebytes_d, _p(Sg), _p(Su), _p(Sd), _p(logits),
                                            stride, nexp_total, topk, x.c(), T, H, F, _p(ids), _p(w), _p(y), _stream(stream)),
          "moe_decode_noalloc")


def moe_decode_scratch_max():
    return _lib.lib().qmm_moe_decode_scratch_max()


def moe_combine_sorted(down, w, kpos, y, T, nexp, E, stream=None):
    """fn.h:38: y[t][d] = sum_e w[t*nexp+e] * down[kpos[t*nexp+e]][d] (E is an argument here)."""
    check(_lib.lib().qmm_moe_combine_sorted(_p(down), _p(w), _p(kpos), _p(y), T, nexp, E, _stream(stream)),
          "moe_combine_sorted")


def moe_silu_quant(gate, up, xq, rows, n, stream=None):
    """fn.h:48: h = silu(g)*u quantised per 32 into xq (XQ8Buf of rows x n)."""
    check(_lib.lib().qmm_moe_silu_quant(_p(gate), _p(up), xq.c(), rows, n, _stream(stream)), "moe_silu_quant")


def f32_gemv(W, x, y, N, K, T, stream=None):
    """fn.h:37: y[t][n] = W[n] . x[t] in f32 (the reference's arithmetic and order)."""
    _dev(W, torch.float32, "W"); _dev(x, torch.float32, "x"); _dev(y, torch.float32, "y")
    check(_lib.lib().qmm_f32_gemv(_p(W), _p(x), _p(y), N, K, T, _stream(stream)), "f32_gemv")


def gemm_f32(A, W, D, M, N, K, stream=None):
    """gemm.h:31 (BlasLt::gemm_f32, the prefill router): D[m][n] = A[m] . W[n] in f32 on the matrix cores."""
    _dev(A, torch.float32, "A"); _dev(W, torch.float32, "W"); _dev(D, torch.float32, "D")
    check(_lib.lib().qmm_gemm_f32(_p(A), _p(W), _p(D), M, N, K, _stream(stream)), "gemm_f32")


def moe_router(Wr, x, logits, ids, w, T, nexp=512, K=None, topk=10, stream=None):
    """qwen4exp.cpp:346-347 in one call: logits = Wr . x (f32_gemv), then moe_route_n on them."""
    _dev(Wr, torch.float32, "Wr"); _dev(x, torch.float32, "x"); _dev(logits, torch.float32, "logits")
    K = x.shape[-1] if K is None else K
    check(_lib.lib().qmm_moe_router(_p(Wr), _p(x), _p(logits), _p(ids), _p(w), T, nexp, K, topk, _stream(stream)),
          "moe_router")


# ---- activation producers (engine/kernels/ops.h) ----
def add_rmsnorm_quant(x, y, w, xn, xq, T, n, eps, stream=None):
    """ops.h:14: per row, x += y (y may be None), xn = rmsnorm(x) * w, xq = q8(xn) (XQ8Buf of T x n)."""
    _dev(x, torch.float32, "x"); _dev(w, torch.float32, "w"); _dev(xn, torch.float32, "xn")
    if y is not None:
        _dev(y, torch.float32, "y")
    check(_lib.lib().qmm_add_rmsnorm_quant(_p(x), 0 if y is None else _p(y), _p(w), _p(xn), xq.c(), T, n, eps,
                                           _stream(stream)), "add_rmsnorm_quant")


def add_rmsnorm_bf16(x, y, w, xb, T, n, eps, stream=None):
    """ops.h:18: per row, x += y (y may be None), xb = bf16(rmsnorm(x) * w) (xb int16/uint16/bfloat16 storage)."""
    _dev(x, torch.float32, "x"); _dev(w, torch.float32, "w")
    if y is not None:
        _dev(y, torch.float32, "y")
    check(_lib.lib().qmm_add_rmsnorm_bf16(_p(x), 0 if y is None else _p(y), _p(w), _p(xb), T, n, eps,
                                          _stream(stream)), "add_rmsnorm_bf16")


def silu_mul_quant(gate, up, xq, n, stream=None):
    """ops.h:24: xq = q8(silu(gate) * up) per 32 over n values."""
    _dev(gate, torch.float32, "gate"); _dev(up, torch.float32, "up")
    check(_lib.lib().qmm_silu_mul_quant(_p(gate), _p(up), xq.c(), n, _stream(stream)), "silu_mul_quant")


def silu_mul_bf16(gate, up, out, n, stream=None):
    """ops.h:20: out = bf16(silu(gate) * up) over n values."""
    _dev(gate, torch.float32, "gate"); _dev(up, torch.float32, "up")
    check(_lib.lib().qmm_silu_mul_bf16(_p(gate), _p(up), _p(out), n, _stream(stream)), "silu_mul_bf16")


# ---- prefill GEMM (engine/kernels/gemm.h) ----
def dequant_bf16(fmt, W, out, N, K, stream=None):
    """gemm.h:12: W -> bf16 [N][K] (out: int16/uint16-sized tensor of N*K elements), bit-exact."""
    _dev(W, torch.uint8, "W")
    check(_lib.lib().qmm_dequant_bf16(fmt, _p(W), _p(out), N, K, _stream(stream)), "dequant_bf16")


def gemm_wq(fmt, W, A, D, M, N, K, stream=None):
    """D[M][N] f32 = A[M][K] bf16 . dequant(W)[N][K]^T, dequantisation fused into the GEMM."""
    _dev(W, torch.uint8, "W"); _dev(A, torch.bfloat16, "A"); _dev(D, torch.float32, "D")
    check(_lib.lib().qmm_gemm_wq(fmt, _p(W), _p(A), _p(D), M, N, K, _stream(stream)), "gemm_wq")


def gemm_bf16(A, W, D, M, N, K, stream=None):
    """BlasLt::gemm (gemm.h:27): D[M][N] bf16 = A[M][K] bf16 . W[N][K]^T bf16, f32 accumulate."""
    _dev(A, torch.bfloat16, "A"); _dev(W, torch.bfloat16, "W"); _dev(D, torch.bfloat16, "D")
    check(_lib.lib().qmm_gemm_bf16(_p(A), _p(W), _p(D), M, N, K, _stream(stream)), "gemm_bf16")


def gemm_bf16_ld(A, lda, W, ldw, D, M, N, K, stream=None):
    """BlasLt::gemm_ld (gemm.h:29): as gemm_bf16 with row strides lda / ldw (elements); A and W may be views."""
    check(_lib.lib().qmm_gemm_bf16_ld(_p(A), lda, _p(W), ldw, _p(D), M, N, K, _stream(stream)), "gemm_bf16_ld")


def f32_to_bf16(x, out, n, stream=None):
    check(_lib.lib().qmm_f32_to_bf16(_p(x), _p(out), n, _stream(stream)), "f32_to_bf16")


def bf16_to_f32(x, out, n, stream=None):
    check(_lib.lib().qmm_bf16_to_f32(_p(x), _p(out), n, _stream(stream)), "bf16_to_f32")


def bf16_to_f32_seg(x, Nt, off, N, out, M, stream=None):
    check(_lib.lib().qmm_bf16_to_f32_seg(_p(x), Nt, off, N, _p(out), M, _stream(stream)), "bf16_to_f32_seg")


def bf16_to_f32_seg2(x, x2, Nt, off, N, out, M, stream=None):
    check(_lib.lib().qmm_bf16_to_f32_seg2(_p(x), _p(x2), Nt, off, N, _p(out), M, _stream(stream)), "bf16_to_f32_seg2")


# ---- MoE prefill ----
MOE_TILE_ROWS = 128    # rows per tile of qmm_moe_gemm_bf16 / qmm_moe_gemm_gate_up_bf16 (at most 128)


def moe_tiles_capacity(T, nslot, nexperts, maxc=MOE_TILE_ROWS):
    return -(-(T * nslot) // maxc) + nexperts + 1


def moe_sort(ids, T, nslot, nexperts, maxc, kpos, rowtok, tiles, counts, stream=None):
    """Device expert sort (replaces the host path of qwen4exp.cpp:628-645).  tiles: int32 [cap][3]."""
    check(_lib.lib().qmm_moe_sort(_p(ids), T, nslot, nexperts, maxc, _p(kpos), _p(rowtok), _p(tiles), _p(counts),
                                  _stream(stream)), "moe_sort")


def moe_gemm_bf16(fmt, shared_fmt, W, Wsh, ebytes, tiles, counts, max_tiles, rowtab, A, D, N, K, stream=None):
    """Grouped expert GEMM over sorted rows, bf16 activations (moe_gemm, gemv.h:49-50)."""
    check(_lib.lib().qmm_moe_gemm_bf16(fmt, shared_fmt, _p(W), _p(Wsh), ebytes, _p(tiles), _p(counts), max_tiles,
                                       _p(rowtab), _p(A), _p(D), N, K, _stream(stream)), "moe_gemm_bf16")


def moe_gemm_gate_up_bf16(fmt, shared_fmt, Wg, Wgsh, Wu, Wush, ebytes, tiles, counts, max_tiles, rowtab, A, H, N, K,
                          stream=None):
    """h = bf16(silu(A . Wg^T) * (A . Wu^T)) over the sorted rows, one launch (gate, up and silu)."""
    check(_lib.lib().qmm_moe_gemm_gate_up_bf16(fmt, shared_fmt, _p(Wg), _p(Wgsh), _p(Wu), _p(Wush), ebytes, _p(tiles),
                                               _p(counts), max_tiles, _p(rowtab), _p(A), _p(H), N, K, _stream(stream)),
          "moe_gemm_gate_up_bf16")


def moe_silu_bf16(gate, up, h, n, stream=None):
    check(_lib.lib().qmm_moe_silu_bf16(_p(gate), _p(up), _p(h), n, _stream(stream)), "moe_silu_bf16")


def moe_gemm(fmt, shared_fmt, W, Wsh, ebytes, tiles, ntiles, stiles, nstiles, ct, rowtab, x, y, N, K, stream=None):
    """moe_gemm (gemv.h:49-50) with the reference's signature: q8 activations (x an XQ8Buf), routed tiles
    tiles[:ntiles] and shared tiles stiles[:nstiles] with host counts; y[k][N] f32, the q8 arithmetic."""
    check(_lib.lib().qmm_moe_gemm_q8(fmt, shared_fmt, _p(W), _p(Wsh), ebytes, _p(tiles), ntiles, _p(stiles), nstiles, ct,
                                     _p(rowtab), x.c(), _p(y), N, K, _stream(stream)), "moe_gemm")
