// ref_gemv_shim.cpp -- exposes the reference's host layout helpers of engine/kernels/gemv.hip
// (wfmt_row_bytes and the load-time row repacks, gemv.hip:1337-1354,1448-1465), compiled from where
// they lie in the reference checkout, through a C ABI: the oracle's restatements of the SoA layouts
// are checked against them byte for byte.  TEST INFRASTRUCTURE ONLY: built into oracle/_ref/
// (git-ignored) by oracle/Makefile, loaded only by tests/ and tests/golden/ on the build host (the
// reference's device code in the same object targets its own GPU and is never launched).
#include "gemv.h"

extern "C" {
size_t refg_wfmt_row_bytes(int f, int K) { return hip::wfmt_row_bytes((hip::WFmt)f, K); }
void refg_repack_row_q6_K(const uint8_t* s, uint8_t* d, int K) { hip::repack_row_q6_K(s, d, K); }
void refg_repack_row_q8_0(const uint8_t* s, uint8_t* d, int K) { hip::repack_row_q8_0(s, d, K); }
void refg_repack_row_q5_1(const uint8_t* s, uint8_t* d, int K) { hip::repack_row_q5_1(s, d, K); }
void refg_repack_row_q5_0(const uint8_t* s, uint8_t* d, int K) { hip::repack_row_q5_0(s, d, K); }
// the experimental interleaved layouts (gemv.hip:1442-1447,1280-1303)
void refg_repack_interleave8(int f, const uint8_t* s, uint8_t* d, int N, int K) { hip::repack_interleave8((hip::WFmt)f, s, d, N, K); }
size_t refg_wmma_il_bytes(int f, int N, int K) { return hip::wmma_il_bytes((hip::WFmt)f, N, K); }
void refg_repack_wmma_il(int f, const uint8_t* s, uint8_t* d, int N, int K) { hip::repack_wmma_il((hip::WFmt)f, s, d, N, K); }
}
