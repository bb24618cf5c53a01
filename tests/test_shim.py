"""CPU check of the drop-in C++ shim (include/hipster_qmm_shim.hpp): it compiles with hipcc against
libhipster_qmm.so, keeps the reference's namespace hip names (engine/kernels/gemv.h, gemm.h, fn.h),
and turns a library error into std::runtime_error instead of the reference's abort()."""
import os
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
HIPCC = "/opt/rocm/bin/hipcc"

SRC = r'''
#include "hipster_qmm_shim.hpp"
#include <cstdio>
int main() {
    // gemv_wmma_ok as the reference's (gemv.hip:1272-1275): not Q5_1_SOA, K % 256 == 0, one K
    hip::GemvSeg seg{hip::WFmt::Q5_1_SOA, nullptr, nullptr, 16, 256};
    hip::GemvSeg ok4[2] = {{hip::WFmt::Q4_K, nullptr, nullptr, 16, 256}, {hip::WFmt::Q5_K, nullptr, nullptr, 16, 256}};
    hip::GemvSeg badk[2] = {{hip::WFmt::Q4_K, nullptr, nullptr, 16, 256}, {hip::WFmt::Q4_K, nullptr, nullptr, 16, 512}};
    if (hip::gemv_wmma_ok(&seg, 1) || !hip::gemv_wmma_ok(ok4, 2) || hip::gemv_wmma_ok(badk, 2)) return 2;
    if (hip::wfmt_row_bytes(hip::WFmt::Q4_K, 5120) != 20 * 144) return 3;
    int caught = 0;
    try {
        hip::gemm_wq(hip::WFmt::Q6_K_SOA, (void*)16, (const uint16_t*)16, (float*)16, 16, 16, 256, nullptr);
    } catch (const std::runtime_error&) { ++caught; }
    try {
        hip::moe_sort((const int*)16, 4, 11, 4096, 64, (int*)16, (int*)16, (hip::MoeTile*)16, (int*)16, nullptr);
    } catch (const std::runtime_error&) { ++caught; }
    try {   // ncol above the fused kernel's limit
        hip::gemv_q8_f32x(hip::WFmt::Q4_K, (void*)16, (const float*)16, (float*)16, 16, 256, 5, nullptr);
    } catch (const std::runtime_error&) { ++caught; }
    try {   // the reference's experimental interleaved layouts are not read here
        hip::gemv_q8(hip::WFmt::Q4_K, (void*)16, hip::XQ8{(int8_t*)16, (float*)16, (float*)16}, (float*)16, 16, 256, 1, 4, 5, nullptr);
    } catch (const std::runtime_error&) { ++caught; }
    try {
        hip::GemvSeg g{hip::WFmt::Q4_K, (void*)16, (float*)16, 16, 256};
        hip::gemv_wmma(&g, 1, hip::XQ8{(int8_t*)16, (float*)16, (float*)16}, 1, 3, nullptr);
    } catch (const std::runtime_error&) { ++caught; }
    try {   // moe_gemm: Q6_K_SOA experts are not a moe_gemm format
        hip::moe_gemm(hip::WFmt::Q6_K_SOA, hip::WFmt::Q8_0_SOA, (void*)16, (void*)16, 1024, (const hip::MoeTile*)16, 1, nullptr, 0,
                      1, nullptr, hip::XQ8{(int8_t*)16, (float*)16, (float*)16}, (float*)16, 16, 256, nullptr);
    } catch (const std::runtime_error&) { ++caught; }
    try {   // gemv_splitk: more splits than 256-weight blocks
        hip::gemv_splitk(hip::WFmt::Q8_0_SOA, (void*)16, hip::XQ8{(int8_t*)16, (float*)16, (float*)16}, (float*)16, 16, 512, 3, 1, nullptr);
    } catch (const std::runtime_error&) { ++caught; }
    try {   // gemm_ld: lda smaller than K
        hip::BlasLt b; b.gemm_ld((const uint16_t*)16, 64, (const uint16_t*)16, 128, (uint16_t*)16, 16, 16, 128, nullptr);
    } catch (const std::runtime_error&) { ++caught; }
    hip::g_persist_blocks = 4; hip::g_moe_tpr = 8;    // the experiment knobs exist (and are ignored)
    if (caught != 8) return 4;
    {   // the load-time repacks of the other formats (gemv.h:16-18), host only
        uint8_t src[34 * 2] = {0}, dst[34 * 2];
        src[0] = 0x00; src[1] = 0x3c;                      // Q8_0 block 0: d = 1
        hip::repack_row_q8_0(src, dst, 64);
        if (dst[64] != 0x00 || dst[65] != 0x3c) return 5;
        uint8_t s5[22] = {0x00, 0x3c}, d5[24];            // Q5_0: d = 1 -> m = -16 (0xcc00)
        hip::repack_row_q5_0(s5, d5, 32);
        if (d5[22] != 0x00 || d5[23] != 0xcc) return 6;
        uint8_t s51[24] = {0}, d51[24];
        hip::repack_row_q5_1(s51, d51, 32);
        if (hip::wfmt_row_bytes(hip::WFmt::Q8_0_SOA, 96) != 102) return 7;
    }
    try {   // a format id the library does not know
        hip::gemv_q8((hip::WFmt)99, (void*)16, hip::XQ8{(int8_t*)16, (float*)16, (float*)16}, (float*)16, 16, 256, 1, 0, 1, nullptr);
    } catch (const std::runtime_error& e) {
        std::printf("%s\n", e.what());
        return 0;
    }
    return 1;
}
'''


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_shim_compiles_and_reports_errors():
    lib = os.path.join(ROOT, "hipster_amd", "lib")
    d = tempfile.mkdtemp()
    try:
        src, exe = os.path.join(d, "t.cpp"), os.path.join(d, "t")
        open(src, "w").write(SRC)
        subprocess.run([HIPCC, "-std=c++17", "-I" + os.path.join(ROOT, "include"), src, "-L" + lib, "-lhipster_qmm",
                        "-Wl,-rpath," + lib, "-o", exe], check=True, capture_output=True)
        r = subprocess.run([exe], capture_output=True, text=True)
        assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
        assert "unsupported weight format" in r.stdout
    finally:
        shutil.rmtree(d, ignore_errors=True)
