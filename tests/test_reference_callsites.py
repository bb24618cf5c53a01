"""The drop-in proof on the CPU: the reference's own engine and validator sources compile against
include/hipster_qmm_shim.hpp, and its two kernel validators link against libhipster_qmm.so.

The reference's engine/ tree is copied to a temporary directory and patched exactly as INTEGRATION.md
prescribes (nothing else changes):
  - kernels/gemv.h and kernels/gemm.h become `#include "hipster_qmm_shim.hpp"`;
  - the declarations of the MoE block of kernels/fn.h (f32_gemv, moe_combine_sorted, moe_route,
    moe_gemv, moe_silu_quant) and of the four producers in kernels/ops.h (add_rmsnorm_quant,
    add_rmsnorm_bf16, silu_mul_quant, silu_mul_bf16) are removed: the shim defines them.
Then every engine source and every bench program that includes those headers is compiled by hipcc for
gfx950 (-fsyntax-only), and engine/bench/bench_gemv.cpp and bench_moe.cpp are built and linked with the
reference's gguf.cpp against the library.  Skipped when the reference checkout is absent.
"""
import concurrent.futures as cf
import os
import re
import shutil
import subprocess
import tempfile

import pytest

from oracle import refpatch

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
HIPCC = refpatch.HIPCC
SOURCES = ["src/qwen4exp.cpp", "src/qwen35.cpp", "src/dflash.cpp", "bench/bench_gemv.cpp", "bench/bench_moe.cpp",
           "bench/batchfn.cpp", "bench/dflash27b.cpp", "bench/prefill27b.cpp", "bench/prefillfn.cpp", "bench/run27b.cpp",
           "bench/runfn.cpp", "bench/spec27b.cpp", "bench/specfn.cpp", "bench/test_fnkernels.cpp"]

pytestmark = pytest.mark.skipif(not (os.path.isdir(refpatch.REF) and os.path.exists(HIPCC)),
                                reason="needs the reference checkout and hipcc")


@pytest.fixture(scope="module")
def patched():
    d = tempfile.mkdtemp()
    yield refpatch.patched_copy(d)
    shutil.rmtree(d, ignore_errors=True)


def _syntax(eng, src):
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-std=c++20", "-fsyntax-only", "-I" + os.path.join(ROOT, "include"),
                        "-Wno-unused-result", os.path.join(eng, src)], capture_output=True, text=True)
    errs = [ln for ln in r.stderr.splitlines() if "error" in ln]
    return src, r.returncode, errs


def test_every_reference_callsite_compiles(patched):
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        res = list(ex.map(lambda s: _syntax(patched, s), SOURCES))
    bad = [(s, e[:5]) for s, rc, e in res if rc != 0]
    assert not bad, bad


def test_call_surface_is_the_shims(patched):
    """Nothing left to forward elsewhere: the patched headers hold no hip:: function declaration on the
    path, and the shim defines every name the engine's removed declarations had."""
    shim = open(os.path.join(ROOT, "include", "hipster_qmm_shim.hpp")).read()
    for n in refpatch.FN_DROP + refpatch.OPS_DROP + ("gemv_splitk", "hc_up_fused", "moe_gemm", "gemv_wmma_q8k", "quantize_x_q8k",
                                   "repack_interleave8", "wmma_il_bytes", "repack_wmma_il", "gemm_ld"):
        assert re.search(r"\b%s\(" % n, shim), n


@pytest.mark.parametrize("bench", ["bench_gemv", "bench_moe"])
def test_reference_validators_link(patched, bench, tmp_path):
    exe = str(tmp_path / bench)
    r = refpatch.build_validator(patched, bench, exe, os.path.join(ROOT, "hipster_amd", "lib"))
    assert r.returncode == 0, r.stderr[-3000:]
    assert os.path.getsize(exe) > 0
