"""The integration patch of INTEGRATION.md applied to a copy of the reference's engine/ tree, and the build
of the reference's two kernel validators (engine/bench/bench_gemv.cpp, bench_moe.cpp) against
libhipster_qmm.so.  TEST INFRASTRUCTURE ONLY: used by tests/test_reference_callsites.py and by
`python oracle/refpatch.py` (called from oracle/Makefile), which writes oracle/_ref/bench_gemv and
oracle/_ref/bench_moe (git-ignored, rpath to hipster_amd/lib relative to the binary, so they run from the
tree copied to the GPU box).  Nothing of the reference is copied into the repository: the patched copy
lives in a temporary directory.

The patch: kernels/gemv.h and kernels/gemm.h become `#include "hipster_qmm_shim.hpp"`; the declarations
of the MoE block of kernels/fn.h and of the four input producers of kernels/ops.h are removed (the shim
defines them).  Nothing else changes.
"""
import os
import re
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
REF = os.environ.get("REF", "/root/reference") + "/engine"
HIPCC = "/opt/rocm/bin/hipcc"
SHIM_LINE = '#pragma once\n#include "hipster_qmm_shim.hpp"\n'
FN_DROP = ("f32_gemv", "moe_combine_sorted", "moe_route", "moe_gemv", "moe_silu_quant")
OPS_DROP = ("add_rmsnorm_quant", "add_rmsnorm_bf16", "silu_mul_quant", "silu_mul_bf16")


def drop_decls(path, names):
    lines = open(path).read().split("\n")
    out, dropped = [], []
    for ln in lines:
        m = re.match(r"^void (\w+)\(", ln)
        if m and m.group(1) in names:
            dropped.append(m.group(1))
            continue
        out.append(ln)
    if sorted(dropped) != sorted(names):
        raise RuntimeError(f"{path}: expected to drop {names}, dropped {dropped}")
    open(path, "w").write("\n".join(out))


def patched_copy(dst_dir):
    """Copy the reference engine/ into dst_dir/engine and apply the integration patch; returns the path."""
    eng = os.path.join(dst_dir, "engine")
    shutil.copytree(REF, eng, ignore=shutil.ignore_patterns("*.o", "build*"))
    for h in ("gemv.h", "gemm.h"):
        open(os.path.join(eng, "kernels", h), "w").write(SHIM_LINE)
    drop_decls(os.path.join(eng, "kernels", "fn.h"), FN_DROP)
    drop_decls(os.path.join(eng, "kernels", "ops.h"), OPS_DROP)
    return eng


def build_validator(eng, bench, out, rpath):
    lib = os.path.join(ROOT, "hipster_amd", "lib")
    return subprocess.run([HIPCC, "--offload-arch=gfx950", "-std=c++20", "-O2", "-I" + os.path.join(ROOT, "include"),
                           os.path.join(eng, "bench", bench + ".cpp"), os.path.join(eng, "src", "gguf.cpp"),
                           "-L" + lib, "-lhipster_qmm", "-Wl,-rpath," + rpath, "-o", out], capture_output=True, text=True)


def main():
    if not os.path.isdir(REF):
        print("reference checkout absent: oracle/_ref validators not rebuilt")
        return 0
    d = tempfile.mkdtemp()
    try:
        eng = patched_copy(d)
        os.makedirs(os.path.join(HERE, "_ref"), exist_ok=True)
        for bench in ("bench_gemv", "bench_moe"):
            out = os.path.join(HERE, "_ref", bench)
            r = build_validator(eng, bench, out, "$ORIGIN/../../hipster_amd/lib")
            if r.returncode != 0:
                sys.stderr.write(r.stderr[-3000:])
                return 1
            print(f"built _ref/{bench}")
    finally:
        shutil.rmtree(d, ignore_errors=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
