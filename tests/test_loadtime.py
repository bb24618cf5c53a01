"""CPU tests of the on-disk side of the path: the GGUF v3 reader (hipster_amd/csrc/gguf_reader.cpp, reference
engine/src/gguf.cpp:71-156) and the load-time layout preparation (hipster_amd/csrc/loadtime.cpp, qwen4exp.cpp:34-65), through the C ABI.

Pins:
  - bytes the reference's own code wrote (tests/golden/loadtime_golden.npz, tests/golden/make_golden.py
    --loadtime): the Q6_K SoA repack, the interleaved layouts, the load-time f32 -> f16 rounding and
    quantize_row_q8_0_soa of F32 / F16 / BF16 rows;
  - GGUF files written by tests/gguf_writer.py (the format spec, independent of both readers): every
    tensor's dims, type, byte count and bytes, the KV values, shard joining, alignment, and the errors
    (bad magic, version 2, truncation, tensor past EOF, missing shard);
  - the reference's own reader on the same files (oracle/_ref/libgguf_ref.so, when built).
"""
import ctypes
import os
import struct

import numpy as np
import pytest

from hipster_amd import _lib, gguf, qmm, synth
from hipster_amd._lib import QmmError
import oracle
from gguf_writer import ARR, BOOL, F32, F64, I8, I16, I32, I64, STR, U8, U16, U32, U64, write_gguf

HERE = os.path.dirname(os.path.abspath(__file__))
G = np.load(os.path.join(HERE, "golden", "loadtime_golden.npz"))


# ---------------------------------------------------------------- load-time layouts vs the reference's bytes
@pytest.mark.parametrize("K", [512, 1280])
def test_q6k_repack_golden(K):
    src, want = G[f"q6k_K{K}_src"], G[f"q6k_K{K}_dst"]
    for r in range(src.shape[0]):
        assert np.array_equal(qmm.repack_row_q6_K(src[r], K), want[r])
    f, got = gguf.prepare_weight(gguf.GType.Q6_K, src, src.shape[0], K)
    assert f == qmm.WFmt.Q6_K_SOA and np.array_equal(got, want)


@pytest.mark.parametrize("name,fmt", [("q4k", synth.Q4_K), ("q5k", synth.Q5_K), ("iq4xs", synth.IQ4_XS)])
def test_interleave8_golden(name, fmt):
    src, want = G[f"il8_{name}_N16_src"], G[f"il8_{name}_N16_dst"]
    assert np.array_equal(qmm.repack_interleave8(fmt, src, 16, 512).reshape(-1), want.reshape(-1))


@pytest.mark.parametrize("name,fmt", [("q4k", synth.Q4_K), ("q5k", synth.Q5_K), ("iq4xs", synth.IQ4_XS),
                                      ("q6ksoa", synth.Q6_K_SOA), ("q8_0soa", synth.Q8_0_SOA)])
@pytest.mark.parametrize("N", [16, 20])
def test_wmma_il_golden(name, fmt, N):
    src, want = G[f"il16_{name}_N{N}_src"], G[f"il16_{name}_N{N}_dst"]
    assert qmm.wmma_il_bytes(fmt, N, 512) == want.size
    assert np.array_equal(qmm.repack_wmma_il(fmt, src, N, 512), want)


def test_layout_errors():
    L = _lib.lib()
    a = np.zeros(144 * 2 * 8, np.uint8)
    assert L.qmm_repack_interleave8(synth.Q6_K_SOA, a.ctypes.data, a.ctypes.data, 8, 512) == -1   # format
    assert L.qmm_repack_interleave8(synth.Q4_K, a.ctypes.data, a.ctypes.data, 7, 512) == -2       # N % 8
    assert L.qmm_wmma_il_bytes(synth.Q5_1_SOA, 16, 512) == 0
    assert L.qmm_wmma_il_bytes(synth.Q4_K, 16, 384) == 0


def test_f16_loadtime_rounding_golden():
    """quantize_row_q8_0_soa's scale goes through quant.h's own f32 -> f16 (round half up, not to even);
    checked through the Q8_0 requantisation of one-block rows whose amax/127 is each test value."""
    x, want = G["f16_in"], G["f16_out"]
    keep = np.isfinite(x) & (np.abs(x) * 127 < 3e38)
    x, want = x[keep], want[keep]
    rows = np.zeros((x.size, 32), np.float32)
    rows[:, 0] = np.abs(x).astype(np.float32) * np.float32(127.0)
    # amax/127 must round back to |x| in f32 for the check to be about the f16 rounding only
    ok = (rows[:, 0] / np.float32(127.0)) == np.abs(x)
    f, got = gguf.prepare_weight(gguf.GType.F32, rows[ok], int(ok.sum()), 32)
    assert f == qmm.WFmt.Q8_0_SOA
    d = got[:, 32:34].copy().view(np.uint16)[:, 0]
    assert np.array_equal(d, want[ok] & 0x7fff), "load-time f16 rounding differs from quant.h"
    assert ok.sum() > 1000


@pytest.mark.parametrize("name,gtype", [("f32", gguf.GType.F32), ("f16", gguf.GType.F16), ("bf16", gguf.GType.BF16)])
def test_q8_0_requant_golden(name, gtype):
    src, want = G[f"q8_0_{name}_src"], G[f"q8_0_{name}_dst"]
    f, got = gguf.prepare_weight(gtype, src.view(np.uint8), src.shape[0], 256, nthreads=3)
    assert f == qmm.WFmt.Q8_0_SOA
    assert np.array_equal(got, want)


def test_prepare_copies_and_repacks():
    """Block formats are copied; Q8_0 / Q5_1 / Q5_0 rows take the pinned row repacks (test_capi)."""
    K, N = 512, 6
    for gt, fmt, f_out in ((gguf.GType.Q4_K, synth.Q4_K, qmm.WFmt.Q4_K), (gguf.GType.Q5_K, synth.Q5_K, qmm.WFmt.Q5_K),
                           (gguf.GType.IQ4_XS, synth.IQ4_XS, qmm.WFmt.IQ4_XS)):
        W = synth.matrix(31, fmt, N, K)
        f, got = gguf.prepare_weight(gt, W, N, K)
        assert f == f_out and np.array_equal(got, W)
    for gt, fmt, fn in ((gguf.GType.Q8_0, synth.Q8_0, qmm.repack_row_q8_0), (gguf.GType.Q5_1, synth.Q5_1, qmm.repack_row_q5_1),
                        (gguf.GType.Q5_0, synth.Q5_0, qmm.repack_row_q5_0)):
        rows = synth.blocks(synth.rng(32 + fmt), fmt, N * K // 32).reshape(N, -1)
        f, got = gguf.prepare_weight(gt, rows, N, K, nthreads=4)
        assert np.array_equal(got, np.stack([fn(rows[r], K) for r in range(N)]))
    with pytest.raises(QmmError):
        gguf.weight_format(gguf.GType.Q3_K, 256)


# ---------------------------------------------------------------- GGUF reader
def _tensors():
    g = synth.rng(40)
    return [
        ("blk.0.ffn_up.weight", 12, (512, 6), synth.matrix(41, synth.Q4_K, 6, 512)),
        ("blk.0.ffn_down.weight", 14, (256, 5), synth.q6k_blocks(g, 5)),
        ("blk.0.attn_q.weight", 8, (64, 3), synth.blocks(g, synth.Q8_0, 6)),
        ("blk.0.ffn_gate_exps.weight", 12, (256, 2, 4), synth.matrix(42, synth.Q4_K, 8, 256)),
        ("token_embd.weight", 1, (32, 2), (g.standard_normal(64) * 0.1).astype(np.float16)),
        ("output_norm.weight", 0, (40,), g.standard_normal(40).astype(np.float32)),
        ("blk.1.attn_v.weight", 7, (96, 2), synth.blocks(g, synth.Q5_1, 6)),
        ("blk.1.attn_k.weight", 6, (32, 3), synth.blocks(g, synth.Q5_0, 3)),
    ]


KV = {"general.architecture": (STR, "qwen35"), "qwen35.block_count": (U32, 64), "qwen35.rope.freq_base": (F32, 1e7),
      "tokenizer.ggml.tokens": (ARR, (STR, ["a", "bb", "ccc"])), "some.i32": (I32, -5), "some.bool": (BOOL, 1),
      "some.u8": (U8, 7), "some.u64": (U64, 1 << 40), "some.arr_u16": (ARR, (U16, [1, 2, 3, 4]))}


def _check(path, tensors, kv):
    with gguf.GGUF(path) as g:
        ts = g.tensors()
        assert [t.name for t in ts] == [t[0] for t in tensors]
        for t, (name, gt, ne, data) in zip(ts, tensors):
            data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
            assert t.type == gt and t.n_dims == len(ne)
            assert t.ne == tuple(list(ne) + [1] * (4 - len(ne)))
            assert t.nbytes == data.size
            assert np.array_equal(t.array(), data)
            assert np.array_equal(g.read_tensor(t), data)
            assert g.get(name) == t
        assert g.arch() == kv["general.architecture"][1]
        assert g.kv_u32("qwen35.block_count") == 64
        assert g.kv_f32("qwen35.rope.freq_base") == np.float32(1e7)
        assert g.kv_u32("some.i32") == (-5) & 0xffffffff
        assert g.kv_u32("some.u8") == 7
        assert g.kv_kind("some.bool") == gguf.KV_BOOL
        assert g.kv_array_len("tokenizer.ggml.tokens") == 3
        assert g.kv_kind("missing") is None and g.find("missing") is None
        with pytest.raises(QmmError):
            g.get("missing")
        with pytest.raises(QmmError):
            g.kv_str("qwen35.block_count")          # wrong kind
        return ts


def test_gguf_roundtrip(tmp_path):
    ts = _tensors()
    p = str(tmp_path / "m.gguf")
    write_gguf(p, ts, KV)
    got = _check(p, ts, KV)
    assert all(t.file_off % 32 == 0 for t in got)


def test_gguf_alignment(tmp_path):
    ts = _tensors()
    p = str(tmp_path / "m.gguf")
    write_gguf(p, ts, KV, alignment=256)
    got = _check(p, ts, KV)
    assert all(t.file_off % 256 == 0 for t in got)


def test_gguf_shards(tmp_path):
    ts = _tensors()
    files = write_gguf(str(tmp_path / "m.gguf"), ts, KV, shards=3)
    assert len(files) == 3
    for f in files:                                 # any shard opens all of them
        got = _check(f, ts, KV)
        assert [t.shard for t in got] == [0, 0, 0, 1, 1, 1, 2, 2]
    with gguf.GGUF(files[1]) as g:
        assert g.kv_u32("split.no") == 0            # split.* keeps the first shard's value
        assert g.mapped_bytes() == sum(os.path.getsize(f) for f in files)
    os.remove(files[2])
    with pytest.raises(QmmError, match="QMM_ERR_IO"):
        gguf.GGUF(files[0])


def test_gguf_errors(tmp_path):
    ts = _tensors()[:3]
    p = str(tmp_path / "m.gguf")
    write_gguf(p, ts, KV)
    raw = open(p, "rb").read()
    cases = {
        "magic": b"GGUX" + raw[4:],
        "version": raw[:4] + struct.pack("<I", 2) + raw[8:],
        "trunc_header": raw[:40],
        "past_eof": raw[:-100],
        "n_dims": None,
    }
    # n_dims = 5 in the first tensor info: find it after the KV block
    first = raw.index(b"blk.0.ffn_up.weight") + len("blk.0.ffn_up.weight")
    cases["n_dims"] = raw[:first] + struct.pack("<I", 5) + raw[first + 4:]
    for name, data in cases.items():
        q = str(tmp_path / f"{name}.gguf")
        open(q, "wb").write(data)
        with pytest.raises(QmmError, match="QMM_ERR_IO"):
            gguf.GGUF(q)
    with pytest.raises(QmmError, match="QMM_ERR_IO"):
        gguf.GGUF(str(tmp_path / "nope.gguf"))
    # an unknown tensor type
    q = str(tmp_path / "type.gguf")
    write_gguf(q, [("t", 99, (32,), np.zeros(32, np.uint8))])
    with pytest.raises(QmmError, match="QMM_ERR_FORMAT"):
        gguf.GGUF(q)


def test_gguf_dims_overflow(tmp_path):
    """Dims whose element count wraps 64 bits (here to 0, so the byte count would be 0 and pass any
    end-of-file check) and an ne[0] beyond int range are refused."""
    for name, ne, gt in (("wrap", (256, 1 << 56, 1 << 8), 12), ("wrap3", (1 << 32, 1 << 32, 1), 0),
                         ("ne0", (1 << 32,), 24)):
        q = str(tmp_path / f"{name}.gguf")
        write_gguf(q, [("t", gt, ne, np.zeros(64, np.uint8))])
        with pytest.raises(QmmError, match="QMM_ERR_IO"):
            gguf.GGUF(q)


def test_gguf_value_types(tmp_path):
    """Every GGUF value type, arrays of strings, nested arrays and an empty array; the tensor after them
    is found at its offset."""
    kv = {"v.i8": (I8, -3), "v.i16": (I16, -300), "v.u16": (U16, 65535), "v.i64": (I64, -(1 << 40)),
          "v.f64": (F64, 2.5), "v.f32": (F32, -0.75), "v.bool": (BOOL, 0), "v.u64": (U64, (1 << 64) - 1),
          "v.strs": (ARR, (STR, ["", "x" * 300])), "v.nest": (ARR, (ARR, [(U8, [1, 2]), (I64, [5])])),
          "v.empty": (ARR, (F64, [])), "v.str": (STR, "")}
    data = np.arange(40, dtype=np.float32)
    p = str(tmp_path / "v.gguf")
    write_gguf(p, [("w", 0, (40,), data)], kv)
    with gguf.GGUF(p) as g:
        assert g.kv_u32("v.i8") == (-3) & 0xffffffff and g.kv_u32("v.i16") == (-300) & 0xffffffff
        assert g.kv_u32("v.u16") == 65535 and g.kv_u32("v.i64") == (-(1 << 40)) & 0xffffffff
        assert g.kv_u32("v.u64") == 0xffffffff and g.kv_u32("v.bool") == 0
        assert g.kv_f32("v.f64") == 2.5 and g.kv_f32("v.f32") == -0.75
        assert g.kv_array_len("v.strs") == 2 and g.kv_array_len("v.nest") == 2 and g.kv_array_len("v.empty") == 0
        assert g.kv_str("v.str") == ""
        assert np.array_equal(g.read_tensor(g.get("w")).view(np.float32), data)
    # an unknown value type inside an array is refused
    raw = open(p, "rb").read()
    at = raw.index(b"v.empty") + len(b"v.empty") + 4          # past the key and the value type (array)
    q = str(tmp_path / "badarr.gguf")
    open(q, "wb").write(raw[:at] + struct.pack("<I", 13) + raw[at + 4:])
    with pytest.raises(QmmError, match="QMM_ERR_IO"):
        gguf.GGUF(q)


def test_gguf_single_shard_name(tmp_path):
    """A -00001-of-00001 name opens that one file; a name with non-digits in the index is a plain file."""
    ts = _tensors()[:2]
    files = write_gguf(str(tmp_path / "m.gguf"), ts, KV, shards=1)
    one = str(tmp_path / "m-00001-of-00001.gguf")
    os.rename(files[0], one)
    _check(one, ts, KV)
    odd = str(tmp_path / "m-0000a-of-00002.gguf")
    write_gguf(odd, ts, KV)
    _check(odd, ts, KV)


@pytest.mark.skipif(oracle.ref_gguf_lib() is None, reason="reference GGUF reader not built (no reference checkout)")
@pytest.mark.parametrize("shards,alignment", [(1, 32), (3, 32), (2, 128)])
def test_gguf_matches_reference_reader(tmp_path, shards, alignment):
    R = oracle.ref_gguf_lib()
    ts = _tensors()
    files = write_gguf(str(tmp_path / "m.gguf"), ts, KV, shards=shards, alignment=alignment)
    h = R.refgg_open(files[-1].encode())
    assert h
    try:
        with gguf.GGUF(files[-1]) as g:
            mine = g.tensors()
            assert R.refgg_n_tensors(h) == len(mine)
            name = ctypes.create_string_buffer(256)
            ne = (ctypes.c_uint64 * 4)()
            typ, shard = ctypes.c_int(), ctypes.c_int()
            nbytes, off = ctypes.c_uint64(), ctypes.c_uint64()
            for i, t in enumerate(mine):
                assert R.refgg_tensor(h, i, name, 256, ne, ctypes.byref(typ), ctypes.byref(nbytes), ctypes.byref(shard),
                                      ctypes.byref(off)) == 0
                assert (name.value.decode(), tuple(ne), typ.value, nbytes.value, shard.value, off.value) == \
                    (t.name, t.ne, t.type, t.nbytes, t.shard, t.file_off)
                buf = np.empty(t.nbytes, np.uint8)
                assert R.refgg_read(h, t.name.encode(), buf.ctypes.data) == 0
                assert np.array_equal(buf, g.read_tensor(t))
            u = ctypes.c_uint32()
            assert R.refgg_kv_u32(h, b"qwen35.block_count", ctypes.byref(u)) == 0 and u.value == g.kv_u32("qwen35.block_count")
            assert R.refgg_kv_u32(h, b"some.i32", ctypes.byref(u)) == 0 and u.value == g.kv_u32("some.i32")
            fl = ctypes.c_float()
            assert R.refgg_kv_f32(h, b"qwen35.rope.freq_base", ctypes.byref(fl)) == 0 and fl.value == g.kv_f32("qwen35.rope.freq_base")
            sb = ctypes.create_string_buffer(64)
            assert R.refgg_kv_str(h, b"general.architecture", sb, 64) == 0 and sb.value.decode() == g.arch()
            if shards > 1:
                assert R.refgg_kv_u32(h, b"split.no", ctypes.byref(u)) == 0 and u.value == g.kv_u32("split.no")
    finally:
        R.refgg_close(h)


@pytest.mark.skipif(oracle.ref_gguf_lib() is None, reason="reference GGUF reader not built (no reference checkout)")
def test_gguf_errors_match_reference(tmp_path):
    """Both readers refuse the same malformed files."""
    R = oracle.ref_gguf_lib()
    p = str(tmp_path / "m.gguf")
    write_gguf(p, _tensors()[:3], KV)
    raw = open(p, "rb").read()
    for name, data in {"magic": b"GGUX" + raw[4:], "version": raw[:4] + struct.pack("<I", 2) + raw[8:],
                       "past_eof": raw[:-100]}.items():
        q = str(tmp_path / f"{name}.gguf")
        open(q, "wb").write(data)
        assert not R.refgg_open(q.encode())
        with pytest.raises(QmmError):
            gguf.GGUF(q)
