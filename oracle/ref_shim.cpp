// ref_shim.cpp -- exposes the reference's own CPU dequantisers (engine/src/quant.h, compiled from
// where they lie under the reference checkout) through a C ABI, so the oracle restatement in
// qmm_oracle.c can be checked against them bit for bit.  TEST INFRASTRUCTURE ONLY: built into
// oracle/_ref/ (git-ignored) by oracle/Makefile, loaded only by tests/ and tests/golden/.
// Compiled with clang++ -O3 and no -march flag, the reference's own build flags
// (engine/CMakeLists.txt:9, build.sh:11), so x86-64 baseline code: no FMA contraction.
#include "quant.h"

#include <thread>
#include <vector>

extern "C" {
float ref_f16_to_f32(uint16_t h) { return hip::f16_to_f32(h); }                       // quant.h:11-17
void ref_get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) { hip::get_scale_min_k4(j, q, d, m); }   // quant.h:37-40
// quant.h:185-201: type 12 = Q4_K, 14 = Q6_K (GGUF type ids)
void ref_dequant_row(int type, const uint8_t* src, float* dst, uint64_t ne0) { hip::dequant_row(type, src, dst, ne0); }
// quant.h:150-155 (the load-time f32 -> f16 rounding) and quant.h:174-183 (F32 rows -> Q8_0 row-SoA)
uint16_t ref_f32_to_f16(float f) { return hip::f32_to_f16(f); }
void ref_quantize_row_q8_0_soa(const float* x, uint8_t* dst, uint64_t K) { hip::quantize_row_q8_0_soa(x, dst, K); }

// The CPU baseline of bench.py: the reference's host GEMV check path (bench_gemv.cpp:95-104 with an f32
// accumulator): per row dequant_row (quant.h:185-201) then a sequential f32 dot with x, rows split over
// nthreads std::threads as the engine's parallel_rows (qwen4exp.cpp:27-31).  The row body is compiled
// for the host's best vector ISA at run time (target_clones), the -march=native equivalent for a
// library built here and run on another host.
// (w: the thread's dequantised row, allocated by the caller: no library templates inside the clones)
__attribute__((target_clones("arch=x86-64-v4", "arch=x86-64-v3", "default")))
static void rows_f32(int type, const uint8_t* W, size_t rb, int K, const float* x, float* y, int r0, int r1, float* w) {
    for (int r = r0; r < r1; ++r) {
        hip::dequant_row(type, W + (size_t)r * rb, w, (uint64_t)K);
        float acc = 0.f;
        for (int k = 0; k < K; ++k) acc += w[k] * x[k];
        y[r] = acc;
    }
}
int ref_gemv_f32_threads(int type, const uint8_t* W, size_t row_bytes, int N, int K, const float* x, float* y, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    std::vector<float> rowbuf((size_t)K * nthreads);
    std::vector<std::thread> th;
    for (int i = 0; i < nthreads; ++i)
        th.emplace_back(rows_f32, type, W, row_bytes, K, x, y, (int)((long long)N * i / nthreads), (int)((long long)N * (i + 1) / nthreads),
                        rowbuf.data() + (size_t)K * i);
    for (auto& t : th) t.join();
    return 0;
}
}
