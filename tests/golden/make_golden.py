"""Writes tests/golden/*.npz from the reference's OWN CPU dequantisers.

The reference (dzannotti/hipster) ships no kernel-level golden vectors, so this script builds them:
it calls engine/src/quant.h (f16_to_f32, get_scale_min_k4, dequant_row for GGUF types 12 = Q4_K and
14 = Q6_K), compiled unchanged from the reference checkout by oracle/Makefile into
oracle/_ref/libqmm_ref.so, on seeded random blocks plus hand-made special blocks, and stores the
inputs and the reference's outputs (quant_golden.npz).  A second file, quant_golden_fmt.npz, holds
the same for the other formats of the call surface -- dequant_row types 13 = Q5_K, 23 = IQ4_XS,
8 = Q8_0, 7 = Q5_1 -- and the bytes the reference's load-time repacks (engine/kernels/gemv.hip:
1351-1354,1448-1465, compiled into oracle/_ref/libqmm_ref_gemv.so) make of seeded Q8_0, Q5_1 and
Q5_0 rows.  Run from the repo root after `make -C oracle`:

    python tests/golden/make_golden.py             # quant_golden.npz
    python tests/golden/make_golden.py --formats   # quant_golden_fmt.npz
    python tests/golden/make_golden.py --loadtime  # loadtime_golden.npz

loadtime_golden.npz holds what the reference's load path writes: repack_row_q6_K rows (gemv.hip:
1341-1350), the experimental interleaved layouts repack_interleave8 / repack_wmma_il (gemv.hip:1280-1303,
1442-1447), the load-time f32 -> f16 rounding (quant.h:150-155) and quantize_row_q8_0_soa of F32, F16
and BF16 rows (quant.h:174-199), all computed by the reference's own code.
"""
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.abspath(os.path.join(HERE, "..", "..")))

import oracle  # noqa: E402
from hipster_amd import synth  # noqa: E402


def f16(v):
    return np.array([v], dtype=np.float16).view(np.uint16)[0]


def q4k_special():
    blocks = []
    z = np.zeros(144, np.uint8); blocks.append(z)                                     # all zero -> 0
    b = np.zeros(144, np.uint8); b[0:2] = np.array([f16(1.0)], np.uint16).view(np.uint8)
    b[4:16] = 0x01; b[16:] = 0x21; blocks.append(b)                                  # known answer: 1.0 / 2.0 runs
    b = np.full(144, 0xFF, np.uint8); b[0:2] = np.array([f16(0.5)], np.uint16).view(np.uint8)
    b[2:4] = np.array([f16(0.25)], np.uint16).view(np.uint8); blocks.append(b)       # scales/mins 63, q 15
    b = synth.q4k_blocks(synth.rng(7), 1)[0].copy(); b[0:2] = [0x01, 0x00]; b[2:4] = [0xff, 0x03]; blocks.append(b)  # subnormal d, dmin
    b = synth.q4k_blocks(synth.rng(8), 1)[0].copy()
    b[0:2] = np.array([f16(-0.0123)], np.uint16).view(np.uint8); b[2:4] = np.array([f16(-0.5)], np.uint16).view(np.uint8)
    blocks.append(b)                                                                  # negative d and dmin
    b = synth.q4k_blocks(synth.rng(9), 1)[0].copy(); b[4:16] = [0xC0, 0x80, 0x40, 0xFF, 0xC0, 0x3F, 0x00, 0x80, 0xF0, 0x0F, 0xA5, 0x5A]
    blocks.append(b)                                                                  # top-bit patterns of the packed scales
    return np.stack(blocks)


def q6k_special():
    blocks = []
    b = np.zeros(210, np.uint8); b[192:208] = 1; b[208:210] = np.array([f16(1.0)], np.uint16).view(np.uint8)
    blocks.append(b)                                                                  # q = 0 everywhere -> -32
    b = np.full(210, 0xFF, np.uint8); b[192:208] = 1; b[208:210] = np.array([f16(1.0)], np.uint16).view(np.uint8)
    blocks.append(b)                                                                  # q = 63 -> 31
    b = synth.q6k_blocks(synth.rng(11), 1)[0].copy(); b[192:208] = 0x80; blocks.append(b)   # int8 scale -128
    b = synth.q6k_blocks(synth.rng(12), 1)[0].copy(); b[208:210] = [0x03, 0x00]; blocks.append(b)  # subnormal d
    b = synth.q6k_blocks(synth.rng(13), 1)[0].copy(); b[208:210] = np.array([f16(-0.75)], np.uint16).view(np.uint8)
    blocks.append(b)                                                                  # negative d
    return np.stack(blocks)


def ref_dequant(ref, gtype, blocks):
    out = np.empty((blocks.shape[0], 256), np.float32)
    for i in range(blocks.shape[0]):
        blk = np.ascontiguousarray(blocks[i])
        ref.ref_dequant_row(gtype, ctypes.c_void_p(blk.ctypes.data), ctypes.c_void_p(out[i].ctypes.data), 256)
    return out


def ref_dequant_n(ref, gtype, blocks, per):
    out = np.empty((blocks.shape[0], per), np.float32)
    for i in range(blocks.shape[0]):
        blk = np.ascontiguousarray(blocks[i])
        ref.ref_dequant_row(gtype, ctypes.c_void_p(blk.ctypes.data), ctypes.c_void_p(out[i].ctypes.data), per)
    return out


def fmt_special(fmt):
    """Edge blocks: zero scale, negative scale, subnormal scale, all-ones quant bytes, all-zero ones."""
    per, nbytes = synth.BLOCK[fmt]
    g = synth.rng(300 + fmt)
    bl = []
    for k in range(5):
        b = synth.blocks(g, fmt, 1)[0].copy()
        if k == 0:
            b[0:2] = 0
        elif k == 1:
            b[0:2] = np.array([f16(-0.03125)], np.uint16).view(np.uint8)
        elif k == 2:
            b[0:2] = [0x05, 0x00]
        elif k == 3:
            b[4 if fmt != Q5_0 else 2:] = 0xFF
        else:
            b[4 if fmt != Q5_0 else 2:] = 0x00
        bl.append(b)
    return np.stack(bl)


Q5_K, IQ4_XS, Q8_0, Q5_1, Q5_0 = synth.Q5_K, synth.IQ4_XS, synth.Q8_0, synth.Q5_1, synth.Q5_0


def main_formats():
    ref, refg = oracle.ref_lib(), oracle.ref_gemv_lib()
    if ref is None or refg is None:
        sys.exit("oracle/_ref libraries not built (needs the reference checkout): make -C oracle")
    out = {}
    for name, fmt, gtype in (("q5k", Q5_K, 13), ("iq4xs", IQ4_XS, 23), ("q8_0", Q8_0, 8), ("q5_1", Q5_1, 7)):
        per = synth.BLOCK[fmt][0]
        bl = np.concatenate([fmt_special(fmt), synth.blocks(synth.rng(20260 + fmt), fmt, 200)])
        out[f"{name}_blocks"] = bl
        out[f"{name}_y"] = ref_dequant_n(ref, gtype, bl, per)
    # load-time repacks of whole rows (K = 512 and K = 96: a K that is not a multiple of 256)
    for name, fmt, fn in (("q8_0", Q8_0, refg.refg_repack_row_q8_0), ("q5_1", Q5_1, refg.refg_repack_row_q5_1),
                          ("q5_0", Q5_0, refg.refg_repack_row_q5_0)):
        for K in (512, 96):
            per, nbytes = synth.BLOCK[fmt]
            rows = synth.blocks(synth.rng(20270 + fmt + K), fmt, 4 * (K // per)).reshape(4, -1)
            if fmt == Q5_0:
                rows.reshape(4, K // per, 22)[0, 0, 0:2] = [0x00, 0x7c]     # d = inf: -16 d overflows
                rows.reshape(4, K // per, 22)[0, 1, 0:2] = [0x01, 0x00]     # subnormal d
            dst_bytes = K // 32 * 24 if fmt != Q8_0 else K + K // 16
            dst = np.zeros((4, dst_bytes), np.uint8)
            for r in range(4):
                s = np.ascontiguousarray(rows[r])
                fn(ctypes.c_void_p(s.ctypes.data), ctypes.c_void_p(dst[r].ctypes.data), K)
            out[f"repack_{name}_K{K}_src"] = rows
            out[f"repack_{name}_K{K}_dst"] = dst
    out["row_bytes"] = np.array([[refg.refg_wfmt_row_bytes(f, K) for f in range(6)] for K in (256, 512, 5120, 17408)],
                                dtype=np.int64)
    np.savez_compressed(os.path.join(HERE, "quant_golden_fmt.npz"), **out)
    print("wrote quant_golden_fmt.npz:", {k: v.shape for k, v in out.items()})


def main_loadtime():
    ref, refg = oracle.ref_lib(), oracle.ref_gemv_lib()
    if ref is None or refg is None:
        sys.exit("oracle/_ref libraries not built (needs the reference checkout): make -C oracle")
    vp = ctypes.c_void_p
    out = {}
    # Q6_K rows -> SoA (K = 512 and 1280)
    for K in (512, 1280):
        rows = synth.q6k_blocks(synth.rng(20300 + K), 3 * (K // 256)).reshape(3, -1)
        dst = np.zeros_like(rows)
        for r in range(3):
            src = np.ascontiguousarray(rows[r])
            refg.refg_repack_row_q6_K(vp(src.ctypes.data), vp(dst[r].ctypes.data), K)
        out[f"q6k_K{K}_src"], out[f"q6k_K{K}_dst"] = rows, dst
    # interleaved layouts: 8-row block interleave (Q4_K, Q5_K, IQ4_XS) and the 16-row piece-major layout
    # (those three plus Q6_K_SOA and Q8_0_SOA rows); N = 16 / 20 (a partial 16-row group), K = 512
    K = 512
    for name, fmt in (("q4k", synth.Q4_K), ("q5k", synth.Q5_K), ("iq4xs", synth.IQ4_XS), ("q6ksoa", synth.Q6_K_SOA),
                      ("q8_0soa", synth.Q8_0_SOA)):
        for N in (16, 20):
            W = np.ascontiguousarray(synth.matrix(20310 + fmt + N, fmt, N, K))
            if fmt in (synth.Q4_K, synth.Q5_K, synth.IQ4_XS) and N % 8 == 0:
                d8 = np.zeros_like(W)
                refg.refg_repack_interleave8(fmt, vp(W.ctypes.data), vp(d8.ctypes.data), N, K)
                out[f"il8_{name}_N{N}_src"], out[f"il8_{name}_N{N}_dst"] = W, d8
            nb = refg.refg_wmma_il_bytes(fmt, N, K)
            d16 = np.zeros(nb, np.uint8)
            refg.refg_repack_wmma_il(fmt, vp(W.ctypes.data), vp(d16.ctypes.data), N, K)
            out[f"il16_{name}_N{N}_src"], out[f"il16_{name}_N{N}_dst"] = W, d16
    # f32 -> f16 at load time: ties, subnormal range, overflow, signed zero, random
    g = synth.rng(20320)
    tie = np.array([1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 2.0 ** -14 * (1 + 2.0 ** -11), 2.0 ** -24 * 1.5, 2.0 ** -25,
                    2.0 ** -25 * 1.0001, 2.0 ** -26, 65504.0, 65519.0, 65520.0, 1e9, 0.0, -0.0, 6.1e-5, 5.96e-8,
                    -1.0 - 2.0 ** -11, 3.0e-6], np.float32)
    f32 = np.concatenate([tie, g.standard_normal(2000).astype(np.float32) * np.float32(10.0) ** g.integers(-9, 5, 2000)])
    out["f16_in"] = f32.astype(np.float32)
    out["f16_out"] = np.array([ref.ref_f32_to_f16(float(v)) for v in out["f16_in"]], np.uint16)
    # quantize_row_q8_0_soa of F32 / F16 / BF16 rows (K = 256, 8 rows; a zero block and large values included)
    K = 256
    x = (g.standard_normal((8, K)) * 3).astype(np.float32)
    x[1, 32:64] = 0
    x[2, :32] *= 1e3
    x[3, 64:96] = 1e-6
    src16 = x.astype(np.float16).view(np.uint16)
    srcbf = synth.to_bf16_bits(x)
    for name, gtype, src in (("f32", 0, x), ("f16", 1, src16), ("bf16", 30, srcbf)):
        src = np.ascontiguousarray(src)
        dst = np.zeros((8, K + K // 16), np.uint8)
        row = np.zeros(K, np.float32)
        for r in range(8):
            sr = np.ascontiguousarray(src[r])
            ref.ref_dequant_row(gtype, vp(sr.ctypes.data), vp(row.ctypes.data), K)
            ref.ref_quantize_row_q8_0_soa(vp(row.ctypes.data), vp(dst[r].ctypes.data), K)
        out[f"q8_0_{name}_src"], out[f"q8_0_{name}_dst"] = src, dst
    np.savez_compressed(os.path.join(HERE, "loadtime_golden.npz"), **out)
    print("wrote loadtime_golden.npz:", len(out), "arrays")


def main():
    if "--formats" in sys.argv:
        return main_formats()
    if "--loadtime" in sys.argv:
        return main_loadtime()
    ref = oracle.ref_lib()
    if ref is None:
        sys.exit("oracle/_ref/libqmm_ref.so not built (needs the reference checkout): make -C oracle")
    q4 = np.concatenate([q4k_special(), synth.q4k_blocks(synth.rng(20250), 250)])
    q6 = np.concatenate([q6k_special(), synth.q6k_blocks(synth.rng(20251), 250)])
    q4_y = ref_dequant(ref, 12, q4)
    q6_y = ref_dequant(ref, 14, q6)
    halfs = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f16_tab = np.array([ref.ref_f16_to_f32(int(h)) for h in halfs], dtype=np.float32)
    # get_scale_min_k4 over j = 0..7 for 64 seeded 12-byte scale arrays
    sc_in = synth.rng(20252).integers(0, 256, (64, 12), dtype=np.uint8)
    sc_out = np.empty((64, 8, 2), np.uint8)
    for i in range(64):
        s = np.ascontiguousarray(sc_in[i])
        for j in range(8):
            d = ctypes.c_uint8(); m = ctypes.c_uint8()
            ref.ref_get_scale_min_k4(j, ctypes.c_void_p(s.ctypes.data), ctypes.byref(d), ctypes.byref(m))
            sc_out[i, j] = (d.value, m.value)
    np.savez_compressed(os.path.join(HERE, "quant_golden.npz"), q4k_blocks=q4, q4k_y=q4_y, q6k_blocks=q6, q6k_y=q6_y,
                        f16_bits=halfs, f16_f32=f16_tab, scale_in=sc_in, scale_out=sc_out)
    print("wrote quant_golden.npz:", q4.shape, q6.shape)


if __name__ == "__main__":
    main()
