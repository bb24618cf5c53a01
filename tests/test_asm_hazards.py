"""Wait states around inline-assembly memory instructions (CPU: compiles the kernels to gfx950
assembly and reads it).

The compiler inserts the wait states the ISA requires before a vector memory instruction it emits
itself (5 after a VALU write of an SGPR the instruction reads, 1 after an SALU write of M0 that an
LDS DMA reads), but it cannot see that an inline-assembly block is such an instruction.  The global
-> LDS DMA and the scalar-base stores of these kernels are inline assembly, and once the compiler
spills SGPRs it reloads their base addresses with v_readlane right before them; read stale, such a
base is a garbage address (a kernel that spilled this way faulted the GPU).  Every DMA block
therefore starts with s_nop 4.  These tests check that the compiled code keeps that guard, and that
no vector memory instruction of the file reads an SGPR or M0 written by a VALU instruction within the
5 instructions before it (which also covers the unguarded stores)."""
import os
import re
import subprocess

import pytest

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
CSRC = os.path.join(ROOT, "hipster_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"
FILES = ["moe_prefill.hip", "router.hip"]      # the sources with inline-assembly memory instructions


def device_asm(src, tmp_path):
    out = tmp_path / (os.path.basename(src) + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", "-o", str(out), src]
    subprocess.run(cmd, check=True, capture_output=True)
    return [l.strip() for l in out.read_text().splitlines()]


def sgprs(op):
    op = op.strip()
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", op)
    if m:
        return {f"s{i}" for i in range(int(m.group(1)), int(m.group(2)) + 1)}
    if re.fullmatch(r"s\d+|m0|vcc|vcc_lo|vcc_hi", op):
        return {op}
    return set()


def instructions(lines):
    """(text, inside inline asm) for every instruction line"""
    out, inasm = [], False
    for l in lines:
        if l == ";;#ASMSTART":
            inasm = True
            continue
        if l == ";;#ASMEND":
            inasm = False
            continue
        if not l or l.startswith(";") or l.startswith(".") or l.endswith(":"):
            continue
        out.append((l.split(";")[0].strip(), inasm))
    return out


@pytest.fixture(scope="module", params=FILES)
def asm(request, tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not installed")
    return request.param, device_asm(os.path.join(CSRC, request.param), tmp_path_factory.mktemp("asm"))


def test_inline_asm_memory_blocks_start_with_nop(asm):
    name, lines = asm
    blocks, cur, inasm = [], [], False
    for l in lines:
        if l == ";;#ASMSTART":
            inasm, cur = True, []
        elif l == ";;#ASMEND":
            inasm = False
            blocks.append([x for x in cur if x and not x.startswith(";")])
        elif inasm:
            cur.append(l)
    # the loads (DMA into LDS) carry the guard; the scalar-base stores of the K = 512 grouped GEMM do
    # not (their base is only ever advanced by scalar adds: the second test checks that)
    mem = [b for b in blocks if any(x.startswith(("global_load", "buffer_load")) for x in b)]
    if name == "moe_prefill.hip":
        assert len(mem) > 100
    bad = [b for b in mem if not b[0].startswith("s_nop 4")]
    assert not bad, bad[:3]


def test_no_valu_sgpr_write_before_vector_memory(asm):
    name, lines = asm
    ins = instructions(lines)
    bad = []
    for k, (text, _) in enumerate(ins):
        op = text.split(None, 1)
        if not op or not op[0].startswith(("global_", "buffer_")):
            continue
        reads = set()
        if len(op) > 1:
            for o in op[1].split(",")[1:]:
                reads |= sgprs(o)
        if "lds" in op[0]:
            reads.add("m0")
        # wait states between a VALU SGPR write and this instruction: one per instruction, s_nop n = n + 1
        ws = 0
        for j in range(k - 1, max(-1, k - 8), -1):
            t = ins[j][0].split(None, 1)
            if t and t[0] == "s_nop":
                ws += int(t[1]) + 1
                continue
            if t and t[0].startswith("v_") and len(t) > 1:
                dst = sgprs(t[1].split(",")[0])
                if dst & reads and ws < 5:
                    bad.append((ins[j][0], text, ws))
            ws += 1
            if ws >= 5:
                break
    assert not bad, bad[:5]
