"""GGUF v3 weights for the kernels: the reference's reader (hip::GGUF, engine/src/gguf.h:43-76) and its
load-time layout choice (to_lin / upload_lin, engine/src/qwen4exp.cpp:34-65, qwen35.cpp:31-58), over the
C ABI of libhipster_qmm.so (qmm_gguf_*, qmm_weight_format, qmm_prepare_weight).

    g = GGUF("model-00001-of-00003.gguf")           # any shard opens all of them
    t = g.get("blk.0.ffn_down.weight")               # GTensor: name, type, ne, nbytes, raw bytes (mmap)
    w = upload_lin(g, "blk.0.ffn_down.weight")       # Lin: fmt, device weight in the kernels' layout, N, K

Errors raise QmmError (the reference throws std::runtime_error).
"""
import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import GgufTensor, QmmError, check

# ggml tensor types (the reference's GType numbering, gguf.h:12-17)
GType = type("GType", (), dict(F32=0, F16=1, Q4_0=2, Q4_1=3, Q5_0=6, Q5_1=7, Q8_0=8, Q8_1=9, Q2_K=10, Q3_K=11, Q4_K=12,
                               Q5_K=13, Q6_K=14, Q8_K=15, IQ4_NL=20, IQ3_S=21, IQ4_XS=23, I8=24, I32=26, BF16=30))
KV_UINT, KV_INT, KV_FLOAT, KV_BOOL, KV_STRING, KV_ARRAY = range(6)


def gtype_block(t):
    """(elements, bytes) per block of a ggml type (gguf.h:20)."""
    bs, tb = ctypes.c_uint32(), ctypes.c_uint32()
    check(_lib.lib().qmm_gtype_block(t, ctypes.byref(bs), ctypes.byref(tb)), "gtype_block")
    return bs.value, tb.value


def gtype_row_bytes(t, ne0):
    bs, tb = gtype_block(t)
    return ne0 // bs * tb


@dataclass
class GTensor:
    """A tensor of the file (gguf.h:26-35); ne[0] is the contiguous (K) dimension."""
    name: str
    type: int
    n_dims: int
    ne: tuple
    nbytes: int
    data: int          # host address inside the read-only mapping
    shard: int
    file_off: int

    def array(self):
        """The raw bytes as a read-only numpy view of the mapping (valid while the GGUF is open)."""
        buf = (ctypes.c_uint8 * self.nbytes).from_address(self.data)
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a


def _tensor(c):
    return GTensor(c.name.decode(), c.type, c.n_dims, tuple(c.ne), c.nbytes, c.data or 0, c.shard, c.file_off)


class GGUF:
    """An opened model: one file, or every shard of <base>-0000i-of-0000N.gguf (gguf.cpp:71-84)."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        check(_lib.lib().qmm_gguf_open(str(path).encode(), ctypes.byref(h)), f"GGUF({path})")
        self._h = h

    def close(self):
        if self._h:
            _lib.lib().qmm_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def tensors(self):
        L = _lib.lib()
        out = []
        for i in range(L.qmm_gguf_n_tensors(self._h)):
            c = GgufTensor()
            check(L.qmm_gguf_tensor_at(self._h, i, ctypes.byref(c)), "tensor_at")
            out.append(_tensor(c))
        return out

    def find(self, name):
        c = GgufTensor()
        st = _lib.lib().qmm_gguf_find(self._h, name.encode(), ctypes.byref(c))
        if st == -9:
            return None
        check(st, "find")
        return _tensor(c)

    def get(self, name):
        t = self.find(name)
        if t is None:
            raise QmmError(f"gguf: missing tensor {name}")
        return t

    def has(self, name):
        return self.find(name) is not None

    def mapped_bytes(self):
        return _lib.lib().qmm_gguf_mapped_bytes(self._h)

    def kv_kind(self, key):
        k = ctypes.c_int()
        st = _lib.lib().qmm_gguf_kv_kind(self._h, key.encode(), ctypes.byref(k))
        return None if st == -9 else (check(st, key), k.value)[1]

    def kv_u32(self, key):
        v = ctypes.c_uint32()
        check(_lib.lib().qmm_gguf_kv_u32(self._h, key.encode(), ctypes.byref(v)), f"kv_u32({key})")
        return v.value

    def kv_f32(self, key):
        v = ctypes.c_float()
        check(_lib.lib().qmm_gguf_kv_f32(self._h, key.encode(), ctypes.byref(v)), f"kv_f32({key})")
        return v.value

    def kv_str(self, key):
        v = ctypes.c_char_p()
        check(_lib.lib().qmm_gguf_kv_str(self._h, key.encode(), ctypes.byref(v)), f"kv_str({key})")
        return v.value.decode()

    def kv_array_len(self, key):
        v = ctypes.c_uint64()
        check(_lib.lib().qmm_gguf_kv_array_len(self._h, key.encode(), ctypes.byref(v)), f"kv_array_len({key})")
        return v.value

    def arch(self):
        return self.kv_str("general.architecture")

    def read_tensor(self, t):
        """The tensor's bytes read with pread into a new host array (gguf.cpp:148-156)."""
        name = t.name if isinstance(t, GTensor) else t
        nbytes = (t if isinstance(t, GTensor) else self.get(name)).nbytes
        out = np.empty(nbytes, np.uint8)
        check(_lib.lib().qmm_gguf_read_tensor(self._h, name.encode(), out.ctypes.data, nbytes), f"read_tensor({name})")
        return out


def weight_format(gtype, K):
    """(WFmt the kernels read, row bytes) for a GGUF weight type (qwen4exp.cpp:34-65)."""
    f, rb = ctypes.c_int(), ctypes.c_size_t()
    check(_lib.lib().qmm_weight_format(gtype, K, ctypes.byref(f), ctypes.byref(rb)), "weight_format")
    return f.value, rb.value


def prepare_weight(gtype, src, N, K, nthreads=8):
    """N rows of a GGUF weight (bytes) -> the kernels' layout (copy, row repack or Q8_0 requantisation)."""
    f, rb = weight_format(gtype, K)
    src = np.ascontiguousarray(src).reshape(-1).view(np.uint8)     # the raw bytes, whatever the dtype
    if src.nbytes < N * gtype_row_bytes(gtype, K):
        raise QmmError("prepare_weight: source shorter than N rows")
    dst = np.empty(N * rb, np.uint8)
    check(_lib.lib().qmm_prepare_weight(gtype, src.ctypes.data, N, K, dst.ctypes.data, nthreads), "prepare_weight")
    return f, dst.reshape(N, rb)


@dataclass
class Lin:
    """A weight ready for the kernels (the reference's Lin / FnLin, qwen35.h:27, qwen4exp.h:30)."""
    fmt: int
    w: object           # torch uint8 tensor [N][row bytes] on the device
    N: int
    K: int
    bytes: int


def upload_lin(g, name, device="cuda", nthreads=8):
    """Read a 2-D weight (or a 3-D expert stack, rows = ne[1]*ne[2]), put it in the kernels' layout and copy
    it to the device (the reference's upload_lin / to_lin)."""
    import torch
    t = g.get(name)
    K, N = int(t.ne[0]), int(t.ne[1] * t.ne[2] * t.ne[3])
    raw = g.read_tensor(t)
    fmt, rows = prepare_weight(t.type, raw, N, K, nthreads)
    w = torch.from_numpy(rows).to(device)
    return Lin(fmt, w, N, K, rows.nbytes)
