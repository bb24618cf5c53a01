// ref_shim.cpp -- exposes the reference's own CPU dequantisers (engine/src/quant.h, compiled from
// where they lie under the reference checkout) through a C ABI, so the oracle restatement in
// qmm_oracle.c can be checked against them bit for bit.  TEST INFRASTRUCTURE ONLY: built into
// oracle/_ref/ (git-ignored) by oracle/Makefile, loaded only by tests/ and tests/golden/.
// Compiled with clang++ -O3 and no -march flag, the reference's own build flags
// (engine/CMakeLists.txt:9, build.sh:11), so x86-64 baseline code: no FMA contraction.
#include "quant.h"

extern "C" {
float ref_f16_to_f32(uint16_t h) { return hip::f16_to_f32(h); }                       // quant.h:11-17
void ref_get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) { hip::get_scale_min_k4(j, q, d, m); }   // quant.h:37-40
// quant.h:185-201: type 12 = Q4_K, 14 = Q6_K (GGUF type ids)
void ref_dequant_row(int type, const uint8_t* src, float* dst, uint64_t ne0) { hip::dequant_row(type, src, dst, ne0); }
// quant.h:150-155 (the load-time f32 -> f16 rounding) and quant.h:174-183 (F32 rows -> Q8_0 row-SoA)
uint16_t ref_f32_to_f16(float f) { return hip::f32_to_f16(f); }
void ref_quantize_row_q8_0_soa(const float* x, uint8_t* dst, uint64_t K) { hip::quantize_row_q8_0_soa(x, dst, K); }
}
