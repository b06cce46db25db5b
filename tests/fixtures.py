"""Parsers for the reference's golden fixtures (copied under tests/golden/ref/).

Each parser follows the reader in the reference test that consumes the file:
  quants_ref.bin / quants_ref_fp4.bin  quants.rs:791-860, :940-1010 (SECT / SRAW)
  mulmat_ref*.bin                      vec_dot.rs:2246-2280 (VMM1)
  q4k_repack_ref.bin, q4_0_repack_ref  repack.rs:5636-5676, :6046-6086
  repack_ref.bin (MXFP4)               repack.rs:5010-5055
  tiled_ref.bin                        tiled.rs:2020-2090 (VMT1)
  *_goss_ref.bin, *_granite_ref.bin    vec_dot.rs:2730-2770 (real-weight dumps)
"""
import os
import struct

import numpy as np

REF_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref")


def path(name):
    return os.path.join(REF_DIR, name)


def read(name):
    with open(path(name), "rb") as f:
        return f.read()


def ref_input(n):
    """The LCG of parity/ref_quants_dump.c (quants.rs:779-788)."""
    out = np.empty(n, dtype=np.float32)
    state = 0x12345678
    for i in range(n):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        s = state - (1 << 32) if state >= (1 << 31) else state
        out[i] = np.float32(np.float32(np.float32(s) / np.float32(1 << 30)) * np.float32(0.75)) - np.float32(0.125)
    return out


def quant_sections(name):
    """[(magic, type_id, n, qbytes, deq f32)] until the 0xFFFF end marker."""
    b = read(name)
    o = 0
    out = []
    while True:
        (magic,) = struct.unpack_from("<I", b, o)
        o += 4
        if magic == 0xFFFF:
            break
        tid, n, qlen = struct.unpack_from("<IQQ", b, o)
        o += 20
        q = np.frombuffer(b, dtype=np.uint8, count=qlen, offset=o).copy()
        o += qlen
        deq = np.frombuffer(b[o:o + 4 * n], dtype=np.float32).copy()
        o += 4 * n
        out.append((magic, tid, n, q, deq))
    return out


def mulmat_sections(name):
    """VMM1 sections: [(type_id, n, rows, cols, xq, y[cols, n], dst[cols, rows])]."""
    from oracle_lib import row_size, BLOCK
    b = read(name)
    o = 0
    out = []
    while True:
        (magic,) = struct.unpack_from("<I", b, o)
        o += 4
        if magic == 0xFFFFFFFF:
            break
        assert magic == 0x314D4D56
        tid, n, rows, cols = struct.unpack_from("<4I", b, o)
        o += 16
        if tid in BLOCK:
            xl = row_size(tid, n) * rows
        elif tid in (0,):
            xl = 4 * n * rows
        elif tid in (1, 30):
            xl = 2 * n * rows
        else:
            xl = {3: 20, 6: 22, 7: 24, 10: 84, 11: 110, 13: 176}[tid] * (n // (256 if tid >= 10 else 32)) * rows
        xq = np.frombuffer(b, dtype=np.uint8, count=xl, offset=o).copy()
        o += xl
        y = np.frombuffer(b, dtype=np.float32, count=n * cols, offset=o).reshape(cols, n).copy()
        o += 4 * n * cols
        dst = np.frombuffer(b, dtype=np.float32, count=rows * cols, offset=o).reshape(cols, rows).copy()
        o += 4 * rows * cols
        out.append((tid, n, rows, cols, xq, y, dst))
    return out


def tiled_sections(name="tiled_ref_kq.bin", kind=0):
    """VMT1 sections (tiled.rs:2020-2090) of one kind.
    kind 0 (MUL_MAT):    [(type_id, n, rows, cols, xq, y [cols, n], dst [cols, rows])]
    kind 1 (MUL_MAT_ID): [(type_id, n, rows, ne11, n_as, n_ids, ne12, xq, y [ne12, ne11, n],
                           ids [ne12, n_ids], dst [ne12, n_ids, rows])]"""
    from oracle_lib import row_size
    b = read(name)
    o = 0
    out = []
    while True:
        (magic,) = struct.unpack_from("<I", b, o)
        o += 4
        if magic == 0xFFFFFFFF:
            break
        assert magic == 0x31544D56
        k, tid, n, rows, cols = struct.unpack_from("<5I", b, o)
        o += 20
        n_as = n_ids = ne12 = 1
        if k == 1:
            n_as, n_ids, ne12 = struct.unpack_from("<3I", b, o)
            o += 12
        xl = row_size(tid, n) * rows * n_as
        xq = np.frombuffer(b, dtype=np.uint8, count=xl, offset=o).copy()
        o += xl
        y = np.frombuffer(b, dtype=np.float32, count=n * cols * ne12, offset=o).copy()
        o += 4 * n * cols * ne12
        if k == 1:
            ids = np.frombuffer(b, dtype=np.int32, count=n_ids * ne12, offset=o).reshape(ne12, n_ids).copy()
            o += 4 * n_ids * ne12
        dst = np.frombuffer(b, dtype=np.float32, count=rows * cols if k == 0 else rows * n_ids * ne12,
                            offset=o).copy()
        o += 4 * dst.size
        if k != kind:
            continue
        if k == 0:
            out.append((tid, n, rows, cols, xq, y.reshape(cols, n), dst.reshape(cols, rows)))
        else:
            out.append((tid, n, rows, cols, n_as, n_ids, ne12, xq.reshape(n_as, rows, -1),
                        y.reshape(ne12, cols, n), ids, dst.reshape(ne12, n_ids, rows)))
    return out


def real_weight_dump(name):
    """parity/{q4k_goss,q4k_granite,q6k_granite,q5_0_goss,q8_0_goss,q5k_real}_ref.bin
    (vec_dot.rs:2730-2770, written by parity/ref_q5k_dump.c): length-prefixed
    sections hdr {type, n, rows, cols, flags}, xq, act f32 [cols, n], plain out,
    repacked weights, repack out, q8k bytes, sgemm out.  flags & 1: the
    reference's production path is the Q4_K 8x8 repack kernel (repack_out),
    else the plain vec_dot (plain)."""
    s = _len_sections(name)
    ty, n, rows, cols, flags = struct.unpack_from("<5I", s[0])
    f32 = lambda v: np.frombuffer(v, dtype=np.float32).copy()
    d = dict(type=ty, n=n, rows=rows, cols=cols, flags=flags,
             xq=np.frombuffer(s[1], dtype=np.uint8).copy(),
             act=f32(s[2]).reshape(cols, n), plain=f32(s[3]).reshape(cols, rows),
             repack_out=f32(s[5]).reshape(cols, rows) if s[5] else None,
             q8k=np.frombuffer(s[6], dtype=np.uint8).copy(),
             sgemm_out=f32(s[7]).reshape(cols, rows) if s[7] else None)
    d["want"] = d["repack_out"] if flags & 1 else d["plain"]
    return d


REAL_WEIGHT_DUMPS = ["q4k_goss_ref.bin", "q4k_granite_ref.bin", "q6k_granite_ref.bin",
                     "q5_0_goss_ref.bin", "q8_0_goss_ref.bin", "q5k_real_ref.bin"]


def _len_sections(name):
    b = read(name)
    o = 0
    secs = []
    while o < len(b):
        (ln,) = struct.unpack_from("<I", b, o)
        o += 4
        secs.append(b[o:o + ln])
        o += ln
    return secs


def repack_dump(name):
    """q4k_repack_ref.bin / q4_0_repack_ref.bin (tagged header) or repack_ref.bin (MXFP4)."""
    s = _len_sections(name)
    hdr = struct.unpack("<%dI" % (len(s[0]) // 4), s[0])
    if name == "repack_ref.bin":
        n, nrows, nr_gemv, nr_gemm, nc = hdr[0:5]
    else:
        n, nrows, nr_gemv, nr_gemm, nc = hdr[1:6]
    u8 = lambda v: np.frombuffer(v, dtype=np.uint8).copy()
    f32 = lambda v: np.frombuffer(v, dtype=np.float32).copy()
    d = dict(n=n, nrows=nrows, nr_gemv=nr_gemv, nr_gemm=nr_gemm, nc=nc,
             src=u8(s[1]), repacked=u8(s[2]), q8=u8(s[3]), q8x4=u8(s[4]),
             gemv=f32(s[5]), gemm=f32(s[6]), gemv_gen=f32(s[7]), gemm_gen=f32(s[8]),
             act_g=f32(s[9]), act_m=f32(s[10]))
    return d


def fa_ref_cases():
    """parity/fa_ref.bin (flash_attn.rs:2064-2117): per case a header of i64
    {mode, dk, dv, h, h_kv, t, s_kv, k_type, v_type} and length-prefixed q, k, v,
    mask, sinks, out, extra (scale, max_bias, softcap)."""
    b = read("fa_ref.bin")
    o = 0
    cases = []

    def nxt():
        nonlocal o
        (ln,) = struct.unpack_from("<I", b, o)
        o += 4
        v = b[o:o + ln]
        o += ln
        return v
    while o < len(b):
        hdr = nxt()
        g = struct.unpack("<%dq" % (len(hdr) // 8), hdr)
        q, k, v, mask, sinks, out, extra = (nxt() for _ in range(7))
        mode, dk, dv, h, h_kv, t, s_kv, kt, vt = g[:9]
        kdt = np.float16 if kt else np.float32
        vdt = np.float16 if vt else np.float32
        sc, mb, cap = struct.unpack("<3f", extra[:12])
        cases.append(dict(
            mode=mode, dk=dk, dv=dv, h=h, h_kv=h_kv, t=t, s=s_kv,
            q=np.frombuffer(q, dtype=np.float32).reshape(h, t, dk),
            k=np.frombuffer(k, dtype=kdt).reshape(h_kv, s_kv, dk),
            v=np.frombuffer(v, dtype=vdt).reshape(h_kv, s_kv, dv),
            mask=np.frombuffer(mask, dtype=np.float16).reshape(t, s_kv) if mask else None,
            sinks=np.frombuffer(sinks, dtype=np.float32) if sinks else None,
            out=np.frombuffer(out, dtype=np.float32).reshape(t, h, dv),
            scale=sc, max_bias=mb, softcap=cap))
    return cases


def fa_probe_groups():
    """parity/fa_probe.bin (flash_attn.rs:2541-2640): record groups
    (geometry, knobs, q, k, v, mask, sinks) followed by 1 + t (+1 if t >= 2)
    records {tag, t index, nth, out}: tag 0 = the T-row batch, tag 1 = row t
    alone, tag 2 = rows 1..T-1."""
    b = read("fa_probe.bin")
    o = 0
    groups = []

    def nxt():
        nonlocal o
        (ln,) = struct.unpack_from("<I", b, o)
        o += 4
        v = b[o:o + ln]
        o += ln
        return v
    while o + 4 <= len(b):
        (magic,) = struct.unpack_from("<I", b, o)
        assert magic == 0xF17E0001
        o += 4
        geom, knobs, q, k, v, m, s = (nxt() for _ in range(7))
        dk, dv, h, h_kv, t, s_kv = struct.unpack("<6q", geom[:48])
        sc, mb, cap = struct.unpack("<3f", knobs[:12])
        recs = []
        for _ in range(1 + t + (1 if t >= 2 else 0)):
            tag, ti, nth = struct.unpack_from("<3I", b, o)
            o += 12
            out = np.frombuffer(nxt(), dtype=np.float32)
            recs.append((tag, ti, nth, out))
        groups.append(dict(
            dk=dk, dv=dv, h=h, h_kv=h_kv, t=t, s=s_kv,
            q=np.frombuffer(q, dtype=np.float32).reshape(h, t, dk),
            k=np.frombuffer(k, dtype=np.float16).reshape(h_kv, s_kv, dk),
            v=np.frombuffer(v, dtype=np.float16).reshape(h_kv, s_kv, dv),
            mask=np.frombuffer(m, dtype=np.float16).reshape(t, s_kv) if m else None,
            sinks=np.frombuffer(s, dtype=np.float32) if s else None,
            scale=sc, max_bias=mb, softcap=cap, recs=recs))
    return groups


# block (elements, bytes) of every type in vecdot3_ref.bin (blocks.rs:14-279)
VDD3_BLOCK = {41: (128, 18), 42: (64, 18), 40: (64, 36), 16: (256, 66), 17: (256, 74), 22: (256, 82),
              18: (256, 98), 21: (256, 110), 19: (256, 50), 29: (256, 56), 20: (32, 18), 23: (256, 136),
              8: (32, 34), 15: (256, 292)}


def vecdot3_sections(name="vecdot3_ref.bin"):
    """VDD3 sections (parity/ref_vecdot_dump3.c): the x86 vec_dot of one
    weight type on LCG block bytes and runtime-quantized activations.
    [(type_id, n, xq bytes, yq bytes (Q8_0 or Q8_K rows), result f32)]"""
    b = read(name)
    o = 0
    out = []
    while True:
        (magic,) = struct.unpack_from("<I", b, o)
        o += 4
        if magic == 0xFFFFFFFF:
            break
        assert magic == 0x33444456
        tid, n = struct.unpack_from("<2I", b, o)
        o += 8
        qk, sz = VDD3_BLOCK[tid]
        xl = n // qk * sz
        vt = 15 if tid in (16, 17, 22, 18, 21, 19, 29, 23) else 8
        yqk, ysz = VDD3_BLOCK[vt]
        yl = n // yqk * ysz
        xq = np.frombuffer(b, dtype=np.uint8, count=xl, offset=o).copy()
        o += xl
        yq = np.frombuffer(b, dtype=np.uint8, count=yl, offset=o).copy()
        o += yl
        (res,) = struct.unpack_from("<f", b, o)
        o += 4
        out.append((tid, n, xq, yq, np.float32(res)))
    return out
