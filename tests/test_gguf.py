"""The library's GGUF reader (ghip_gguf_*; gguf.rs:388-655) on the host.

Pinned by: the reference's own vocab file (its tokenizer tests' fixture,
ggml-vocab-llama-spm.gguf) against the facts vocab.rs:4290-4305 asserts
(32000 tokens, bos 1, eos 2, unk 0, add_bos, no add_eos, token 13 = <0x0A>),
every kv pair of that file against a straight Python reading of the format
(tests/gguf_py.py), and files written here with tensors of several types,
alignments and splits, whose offsets and bytes are known by construction;
plus each error of GgufError (gguf.rs:278-300) with its text.
"""
import os
import struct

import numpy as np
import pytest

import gguf_py as G

HERE = os.path.dirname(os.path.abspath(__file__))
VOCAB = os.path.join(HERE, "golden", "ref", "ggml-vocab-llama-spm.gguf")


def ghip():
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(HERE), "llama.rust_amd"))
    import ghip as g
    return g


def test_reference_vocab_known_answers():
    g = ghip().Gguf(VOCAB)
    assert g.version == 3 and g.n_parts == 1
    toks = g.get("tokenizer.ggml.tokens")
    assert len(toks) == 32000
    assert g.get("tokenizer.ggml.model") == "llama"
    assert g.get_u32("tokenizer.ggml.bos_token_id") == 1
    assert g.get_u32("tokenizer.ggml.eos_token_id") == 2
    assert g.get_u32("tokenizer.ggml.unknown_token_id") == 0
    assert g.get("tokenizer.ggml.add_bos_token") is True
    assert g.get("tokenizer.ggml.add_eos_token") is False
    assert toks[13] == "<0x0A>"
    assert toks[29871] == "▁"  # the SPM space piece (vocab.rs:4380 tokenizes "\xff" to [29871, 258])
    assert g.tensors() == []
    assert g.data_offset == os.path.getsize(VOCAB)  # no tensors: no padding, data section at the end


def test_reference_vocab_every_kv_matches_format_reading():
    g = ghip().Gguf(VOCAB)
    ver, kv, ts, data = G.read(VOCAB)
    assert g.keys() == list(kv)
    for k, v in kv.items():
        got = g.get(k)
        if isinstance(v, float):
            assert got == pytest.approx(v, rel=0, abs=0) or np.float32(got) == np.float32(v), k
        elif isinstance(v, list) and v and isinstance(v[0], float):
            assert np.array_equal(np.float32(got), np.float32(v)), k
        else:
            assert got == v, k


def _tensors(rng):
    out = []
    for name, ty, ne in [("tok_embd.weight", 0, [32, 3]), ("blk.0.attn_q.weight", 12, [512, 4]),
                         ("blk.0.ffn_down.weight", 14, [256, 5]), ("blk.0.ffn_gate_exps.weight", 39, [64, 3, 2]),
                         ("norm", 1, [7])]:
        blck, bs = G.BLOCK[ty]
        n = int(np.prod(ne)) // blck * bs
        out.append((name, ty, ne, rng.integers(0, 256, n, dtype=np.uint8).tobytes()))
    return out


@pytest.mark.parametrize("alignment", [None, 32, 64, 256])
def test_written_file_tensors(tmp_path, alignment):
    rng = np.random.default_rng(alignment or 1)
    kv = [("general.architecture", G.STR, "llama"), ("llama.block_count", G.U32, 1),
          ("llama.rope.freq_base", G.F32, 500000.0), ("some.i64", G.I64, -5), ("some.u64", G.U64, 2 ** 40),
          ("some.arr", G.ARR, (G.I32, [1, -2, 3])), ("some.strs", G.ARR, (G.STR, ["a", "", "ccc"])),
          ("some.bool", G.BOOL, True), ("some.f64", G.F64, 0.25), ("some.u8", G.U8, 200), ("some.i16", G.I16, -7)]
    if alignment:
        kv.append(("general.alignment", G.U32, alignment))
    ts = _tensors(rng)
    path = str(tmp_path / "m.gguf")
    data_start, offs = G.write(path, kv, ts, alignment=alignment or 32)
    g = ghip().Gguf(path)
    assert g.alignment == (alignment or 32)
    assert g.data_offset == data_start and data_start % (alignment or 32) == 0
    info = g.tensors()
    assert [t["name"] for t in info] == [t[0] for t in ts]
    for t, (name, ty, ne, data), off in zip(info, ts, offs):
        blck, bs = G.BLOCK[ty]
        ne4 = ne + [1] * (4 - len(ne))
        nb = [bs, bs * ne4[0] // blck]
        nb += [nb[1] * ne4[1], nb[1] * ne4[1] * ne4[2]]
        assert (t["type"], t["ne"], t["nb"], t["offset"], t["size"], t["part"]) == (ty, ne4, nb, off, len(data), 0)
        assert g.tensor_bytes(name) == data
    assert g.get("some.arr") == [1, -2, 3] and g.get("some.strs") == ["a", "", "ccc"]
    assert g.get("some.i64") == -5 and g.get("some.u64") == 2 ** 40 and g.get("some.bool") is True
    # Value::as_u32 / as_f32 casts (gguf.rs:141-168)
    assert g.get_u32("some.u8") == 200 and g.get_u32("some.i64") is None and g.get_u32("some.u64") is None
    assert g.get_u32("some.i16") == (2 ** 32 - 7)  # `as u32` of a negative i16 wraps
    assert g.get_f32("llama.rope.freq_base") == 500000.0 and g.get_f32("some.i64") == -5.0
    assert g.get_u32("general.architecture") is None


def _raw(path, body):
    with open(path, "wb") as f:
        f.write(body)


def _hdr(nt, nkv, version=3):
    return b"GGUF" + struct.pack("<IQQ", version, nt, nkv)


def _kv(key, ty, v):
    return G._s(key) + struct.pack("<I", ty) + G._val(ty, v)


def _tinfo(name, ne, ty, off=0):
    return G._s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<q", n) for n in ne) + struct.pack("<IQ", ty, off)


ERROR_CASES = [
    (b"GGUX" + b"\0" * 20, "not a GGUF file (bad magic)"),
    (_hdr(0, 0, version=4), "unsupported GGUF version 4 (max 3)"),
    (b"GGUF\3\0", "truncated file while reading version"),
    (_hdr(0, 1) + _kv("a", G.U32, 1)[:-2], "truncated file while reading kv value"),
    (_hdr(0, 1) + G._s("a") + struct.pack("<I", 13), "invalid gguf metadata type 13"),
    (_hdr(0, 1) + G._s("a") + struct.pack("<IIQ", G.ARR, 9, 0), "invalid gguf array element type 9"),
    (_hdr(0, 2) + _kv("a", G.U32, 1) + _kv("a", G.U32, 2), "duplicate key 'a'"),
    (_hdr(0, 1) + _kv("", G.U32, 1), "truncated file while reading empty kv key"),
    (_hdr(0, 1) + _kv("general.alignment", G.U32, 48), "alignment 48 not a power of 2"),
    (_hdr(0, 1) + _kv("general.alignment", G.STR, "x"), "key 'general.alignment' is string, expected uint32"),
    (_hdr(2, 0) + _tinfo("w", [32], 0) + _tinfo("w", [32], 0), "duplicate tensor name 'w'"),
    (_hdr(1, 0) + _tinfo("x" * 64, [32], 0), "tensor name too long: '" + "x" * 64 + "'"),
    (_hdr(1, 0) + _tinfo("w", [1, 1, 1, 1, 1], 0), "tensor 'w' has invalid shape/type"),
    (_hdr(1, 0) + _tinfo("w", [-1], 0), "tensor 'w' has invalid shape/type"),
    (_hdr(1, 0) + _tinfo("w", [32], 5), "tensor 'w' has invalid shape/type"),     # type 5 does not exist
    (_hdr(1, 0) + _tinfo("w", [48], 12), "tensor 'w' has invalid shape/type"),    # 48 % 256 != 0
    (_hdr(1, 0) + _tinfo("w", [32], 0)[:-3], "truncated file while reading tensor offset"),
    # element count 2^64 and byte size 2^66: refused, not wrapped to a small size
    (_hdr(1, 0) + _tinfo("w", [2 ** 32, 2 ** 32], 0), "tensor 'w' has invalid shape/type"),
    (_hdr(1, 0) + _tinfo("w", [2 ** 31, 2 ** 31, 4], 0), "tensor 'w' has invalid shape/type"),
    # an array count the rest of the file cannot hold is refused before any element is built
    (_hdr(0, 1) + G._s("a") + struct.pack("<IIQ", G.ARR, G.U8, 2 ** 40), "truncated file while reading kv value"),
]


@pytest.mark.parametrize("body,msg", ERROR_CASES, ids=[m[:40] for _, m in ERROR_CASES])
def test_errors(tmp_path, body, msg):
    path = str(tmp_path / "bad.gguf")
    _raw(path, body)
    with pytest.raises(ghip().GhipError) as e:
        ghip().Gguf(path)
    assert str(e.value) == msg


def test_missing_file(tmp_path):
    with pytest.raises(ghip().GhipError, match="io error"):
        ghip().Gguf(str(tmp_path / "nope.gguf"))


def _write_splits(tmp_path, n, tensors_count=None, bad_no=None, dup=False):
    rng = np.random.default_rng(3)
    prefix = str(tmp_path / "model")
    allts = []
    for k in range(n):
        ts = [(f"t{k}.{j}", 0, [8, 2], rng.integers(0, 256, 64, dtype=np.uint8).tobytes()) for j in range(2)]
        if dup and k == 2:
            ts[0] = ("t0.0",) + ts[0][1:]
        kv = [("split.no", G.U16, bad_no if (bad_no is not None and k == 1) else k)]
        if k == 0:
            kv = [("general.name", G.STR, "m"), ("split.count", G.U16, n),
                  ("split.tensors.count", G.I32, tensors_count if tensors_count is not None else 2 * n)] + kv
        G.write(f"{prefix}-{k + 1:05d}-of-{n:05d}.gguf", kv, ts)
        allts += ts
    return f"{prefix}-00001-of-{n:05d}.gguf", allts


def test_splits(tmp_path):
    path, allts = _write_splits(tmp_path, 3)
    g = ghip().Gguf(path)
    assert g.n_parts == 3
    info = g.tensors()
    assert [t["name"] for t in info] == [t[0] for t in allts]
    assert [t["part"] for t in info] == [0, 0, 1, 1, 2, 2]
    for name, _, _, data in allts:
        assert g.tensor_bytes(name) == data
    one = ghip().Gguf(path, follow_splits=False)  # open_single ignores split.*
    assert one.n_parts == 1 and len(one.tensors()) == 2


@pytest.mark.parametrize("kw,msg", [
    (dict(tensors_count=5), "corrupted model: 5 tensors expected but 6 found"),
    (dict(bad_no=2), "invalid split file idx: 2"),
    (dict(dup=True), "duplicate tensor name 't0.0'"),
])
def test_split_errors(tmp_path, kw, msg):
    path, _ = _write_splits(tmp_path, 3, **kw)
    with pytest.raises(ghip().GhipError, match=msg):
        ghip().Gguf(path)


def test_split_missing_part(tmp_path):
    path, _ = _write_splits(tmp_path, 3)
    os.remove(str(tmp_path / "model-00003-of-00003.gguf"))
    with pytest.raises(ghip().GhipError, match="failed to load GGUF split from .*model-00003-of-00003.gguf"):
        ghip().Gguf(path)
