"""GPU end of the load path: weights written into a (sharded) GGUF v3 file, opened with the library's
reader, put in the kernels' layout at load (the reference's to_lin, qwen4exp.cpp:34-65), uploaded and run
through the decode GEMV, against the oracle on the same prepared weights (1e-5, the GEMV bar); and the
reference's own kernel validators (engine/bench/bench_moe.cpp and bench_gemv.cpp, built by oracle/refpatch.py
against this library) run on synthetic GGUF expert tensors, their OK / MISMATCH verdicts asserted."""
import os
import re
import subprocess

import numpy as np
import pytest
import torch

import oracle
from hipster_amd import gguf, qmm, synth
from tests.gguf_writer import STR, U32, write_gguf
from tests.gpu_util import host, max_rel_mag

pytestmark = pytest.mark.gpu
ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))


def _f16_rows(seed, N, K):
    return (synth.normal_f32(seed, (N, K)) * 0.02).astype(np.float16)


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    d = tmp_path_factory.mktemp("gguf")
    g = synth.rng(600)
    q5 = synth.blocks(g, synth.Q5_0, 512 * 5120 // 32).reshape(512, -1)
    tensors = [
        ("blk.0.ffn_up.weight", gguf.GType.Q4_K, (5120, 17408), synth.matrix(601, synth.Q4_K, 17408, 5120)),
        ("blk.0.ffn_down.weight", gguf.GType.Q6_K, (17408, 5120), synth.matrix(602, synth.Q6_K, 5120, 17408)),
        ("blk.0.attn_q.weight", gguf.GType.Q8_0, (5120, 1024), synth.blocks(g, synth.Q8_0, 1024 * 160)),
        ("blk.0.attn_k.weight", gguf.GType.F16, (5120, 256), _f16_rows(603, 256, 5120)),
        ("blk.0.attn_v.weight", gguf.GType.Q5_0, (5120, 512), q5),
        ("blk.0.ffn_gate.weight", gguf.GType.IQ4_XS, (2048, 640), synth.matrix(604, synth.IQ4_XS, 640, 2048)),
    ]
    files = write_gguf(str(d / "m.gguf"), tensors, {"general.architecture": (STR, "qwen35"), "qwen35.block_count": (U32, 1)},
                       shards=3)
    return files, {t[0]: t for t in tensors}


@pytest.mark.parametrize("name", ["blk.0.ffn_up.weight", "blk.0.ffn_down.weight", "blk.0.attn_q.weight",
                                  "blk.0.attn_k.weight", "blk.0.attn_v.weight", "blk.0.ffn_gate.weight"])
def test_loaded_weight_gemv(gpu, model, name):
    files, tabs = model
    print(f"gguf gemv {name}", flush=True)
    with gguf.GGUF(files[1]) as g:
        lin = gguf.upload_lin(g, name)
        t = g.get(name)
        src = g.read_tensor(t)
    _, gt, ne, _ = tabs[name]
    K, N = ne
    assert (lin.N, lin.K) == (N, K) and t.type == gt
    f_want, rows = gguf.prepare_weight(gt, src, N, K)
    assert lin.fmt == f_want
    assert np.array_equal(host(lin.w), rows)                   # the upload is the prepared layout
    M = 3
    x = synth.normal_f32(610 + K, (M, K))
    xb = qmm.XQ8Buf(M, K)
    qmm.quantize_x_q8(torch.from_numpy(x).cuda(), xb, M, K)
    y = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    qmm.gemv_q8(lin.fmt, lin.w, xb, y, N, K, M)
    q, d, _ = oracle.quantize_x_q8(x)
    sel = np.unique(np.linspace(0, N - 1, 256).astype(np.int32))
    ref, mag = oracle.gemv_ref_rows(lin.fmt, rows, N, K, oracle.q8_to_f32(q, d), sel)
    assert max_rel_mag(host(y)[:, sel], ref, mag) < 1e-5


BENCH_MOE = os.path.join(ROOT, "oracle", "_ref", "bench_moe")


@pytest.mark.skipif(not os.path.exists(BENCH_MOE), reason="reference validator not built (needs the reference checkout)")
@pytest.mark.parametrize("fmt,gt", [(synth.Q4_K, gguf.GType.Q4_K), (synth.Q8_0, gguf.GType.Q8_0)])
def test_reference_bench_moe_validates(gpu, tmp_path, fmt, gt):
    """engine/bench/bench_moe.cpp as the reference wrote it: T tokens x 10 random experts, slots sorted on the
    host into tiles of 16*ct columns, moe_gemm (q8 activations) through the shim, 8 outputs checked against
    its own CPU dequant . x; prints OK or MISMATCH per ct."""
    E, N, K = 64, 512, 2048
    W = synth.blocks(synth.rng(620 + fmt), fmt, E * N * K // synth.BLOCK[fmt][0])
    p = str(tmp_path / "e.gguf")
    write_gguf(p, [("blk.0.ffn_gate_exps.weight", gt, (K, N, E), W)])
    print(f"bench_moe fmt={fmt}", flush=True)
    r = subprocess.run([BENCH_MOE, p, "blk.0.ffn_gate_exps.weight", "512"], capture_output=True, text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    lines = [ln for ln in r.stdout.splitlines() if "CT=" in ln]
    assert len(lines) == 3 and all(re.search(r"maxrel \S+ OK", ln) for ln in lines), lines


BENCH_GEMV = os.path.join(ROOT, "oracle", "_ref", "bench_gemv")
GEMV_LINE = re.compile(r"ncol=(\d+) tpr=\s*(\d+) rpt=(\d+): .* err_vs_ref=(\S+) (OK|MISMATCH)")


@pytest.mark.skipif(not os.path.exists(BENCH_GEMV), reason="reference validator not built (needs the reference checkout)")
@pytest.mark.parametrize("fmt,gt", [(synth.Q8_0, gguf.GType.Q8_0), (synth.Q5_1, gguf.GType.Q5_1)])
def test_reference_bench_gemv_validates(gpu, tmp_path, fmt, gt):
    """engine/bench/bench_gemv.cpp as the reference wrote it, on an expert tensor of the engine's K = 640
    (rows repacked to SoA by the validator itself): every tpr / rpt configuration it runs at 1..8 columns
    through gemv_q8, each checked on 64 sampled rows against its own CPU dequant . x (OK below 1e-5), then
    its decode gather (gemv_moe, x rows per slot) timed.  The validator stops at the first call the
    library refuses, so the count of lines is asserted too."""
    E, N, K = 8, 512, 640
    W = synth.blocks(synth.rng(630 + fmt), fmt, E * N * K // synth.BLOCK[fmt][0])
    p = str(tmp_path / "e.gguf")
    write_gguf(p, [("blk.0.ffn_down_exps.weight", gt, (K, N, E), W)])
    print(f"bench_gemv fmt={fmt}", flush=True)
    r = subprocess.run([BENCH_GEMV, p, "blk.0.ffn_down_exps.weight", "8", "q8"], capture_output=True, text=True,
                       timeout=300)
    print(r.stdout[-3000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    got = [GEMV_LINE.search(ln) for ln in r.stdout.splitlines() if "err_vs_ref" in ln]
    # K % 256 != 0: the 3xx configurations are skipped; ncol 1 runs tpr 32..1 and 8/4 with rpt 3,
    # ncol 2, 3, 4, 8 run tpr 32 and 4 and 4 with rpt 3
    assert len(got) == 8 + 4 * 3 and all(got), r.stdout
    assert all(m.group(5) == "OK" for m in got), r.stdout
    assert "moe tpr= 1:" in r.stdout
