"""GGUF v3 writer for the tests (the reader under test is hipster_amd/csrc/gguf_reader.cpp; the reference's own
reader, engine/src/gguf.cpp, only reads).

Layout written (ggml's GGUF v3): magic "GGUF", version 3, n_tensors u64, n_kv u64; the KV pairs (key
string, value type u32, value); the tensor infos (name string, n_dims u32, ne[n_dims] u64, ggml type
u32, offset u64 relative to the data section); zero padding to `alignment`; the tensor data, each
tensor starting at a multiple of `alignment`.  Strings are u64 length + bytes.

write_gguf(path, tensors, kv, shards=n) with n > 1 writes <base>-0000i-of-0000N.gguf, tensors split
over the shards in order, every shard carrying the KV pairs plus split.no / split.count /
split.tensors.count (llama.cpp's split convention).
"""
import struct

import numpy as np

# GGUF value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q", I64: "<q",
        F64: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v):
    if vtype == STR:
        return _str(v)
    if vtype == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[vtype], v)


def _file(path, kv, tensors, alignment):
    head = [b"GGUF", struct.pack("<IQQ", 3, len(tensors), len(kv))]
    for key, (vtype, v) in kv.items():
        head.append(_str(key) + struct.pack("<I", vtype) + _value(vtype, v))
    offs, off = [], 0
    for name, gtype, ne, data in tensors:
        offs.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    for (name, gtype, ne, data), o in zip(tensors, offs):
        head.append(_str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne) +
                    struct.pack("<IQ", gtype, o))
    h = b"".join(head)
    with open(path, "wb") as f:
        f.write(h)
        f.write(b"\0" * ((-len(h)) % alignment))
        pos = 0
        for (name, gtype, ne, data), o in zip(tensors, offs):
            f.write(b"\0" * (o - pos))
            f.write(data)
            pos = o + len(data)


def write_gguf(path, tensors, kv=None, shards=1, alignment=32):
    """tensors: list of (name, ggml type, ne tuple (ne[0] contiguous), bytes-like data).  kv: {key: (type, value)}
    (ARR values are (element type, list)).  Returns the list of files written."""
    kv = dict(kv or {})
    if alignment != 32:
        kv["general.alignment"] = (U32, alignment)
    tensors = [(n, t, tuple(int(x) for x in ne), bytes(np.ascontiguousarray(d).view(np.uint8).tobytes()))
               for n, t, ne, d in tensors]
    if shards == 1:
        _file(path, kv, tensors, alignment)
        return [path]
    assert path.endswith(".gguf")
    base = path[:-5]
    per = -(-len(tensors) // shards)
    files = []
    for i in range(shards):
        part = tensors[i * per:(i + 1) * per]
        skv = dict(kv)
        skv["split.no"] = (U16, i)
        skv["split.count"] = (U16, shards)
        skv["split.tensors.count"] = (I32, len(tensors))
        p = f"{base}-{i + 1:05d}-of-{shards:05d}.gguf"
        _file(p, skv, part, alignment)
        files.append(p)
    return files
