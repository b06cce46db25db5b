"""Test infrastructure: a plain GGUF v3 writer and reader in Python, from the
format (gguf.rs:1-4: magic, version, counts, kv pairs, tensor infos, the
aligned data section; little-endian), used to build files for the library's
reader and to cross-read them.  Not part of the product."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}
# block size, bytes per block (the ggml types the tests write)
BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 14: (256, 210), 39: (32, 17)}


def _s(x):
    b = x.encode() if isinstance(x, str) else x
    return struct.pack("<Q", len(b)) + b


def _val(ty, v):
    if ty == STR:
        return _s(v)
    if ty == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_val(et, x) for x in items)
    return struct.pack(_FMT[ty], v)


def write(path, kv, tensors, alignment=32, version=3, raw_tail=b""):
    """kv: [(key, type, value)], arrays as (elem_type, [values]);
    tensors: [(name, ggml_type, ne list, data bytes)].  Data laid out in
    order, each tensor at a multiple of `alignment`."""
    out = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv))
    for k, ty, v in kv:
        out += _s(k) + struct.pack("<I", ty) + _val(ty, v)
    offs, cur = [], 0
    for name, ty, ne, data in tensors:
        cur = (cur + alignment - 1) // alignment * alignment
        offs.append(cur)
        cur += len(data)
    for (name, ty, ne, data), off in zip(tensors, offs):
        out += _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<q", n) for n in ne)
        out += struct.pack("<IQ", ty, off)
    if tensors:
        out += b"\0" * ((-len(out)) % alignment)
    data_start = len(out)
    blob = bytearray(cur)
    for (name, ty, ne, data), off in zip(tensors, offs):
        blob[off:off + len(data)] = data
    out += bytes(blob) + raw_tail
    with open(path, "wb") as f:
        f.write(out)
    return data_start, offs


def read(path):
    """(version, {key: value}, [(name, type, ne, offset)], data_offset) by a
    straight reading of the format."""
    b = open(path, "rb").read()
    o = 0

    def take(fmt):
        nonlocal o
        v = struct.unpack_from(fmt, b, o)
        o += struct.calcsize(fmt)
        return v[0]

    def string():
        nonlocal o
        n = take("<Q")
        s = b[o:o + n]
        o += n
        return s.decode("utf-8", errors="surrogateescape")

    def value(ty):
        if ty == STR:
            return string()
        if ty == ARR:
            et, n = take("<I"), take("<Q")
            return [value(et) for _ in range(n)]
        return take(_FMT[ty])

    assert b[:4] == b"GGUF"
    o = 4
    ver, nt, nkv = take("<I"), take("<Q"), take("<Q")
    kv = {}
    for _ in range(nkv):
        k = string()
        kv[k] = value(take("<I"))
    ts = []
    for _ in range(nt):
        name = string()
        nd = take("<I")
        ne = [take("<q") for _ in range(nd)] + [1] * (4 - nd)
        ty, off = take("<I"), take("<Q")
        ts.append((name, ty, ne, off))
    al = kv.get("general.alignment", 32)
    data = (o + al - 1) // al * al if nt else o
    return ver, kv, ts, data
