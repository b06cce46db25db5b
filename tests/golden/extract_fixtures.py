"""Copy the reference's committed parity fixtures for the quantized hot path.

The files under ``parity/`` of fly88oj/llama.rust (MIT licence, copyright 2026
fly88oj) are golden vectors that an instrumented llama.cpp build produced.  They
are data (inputs and expected outputs), copied verbatim -- except
``tiled_ref.bin``, of which only the Q4_K, Q5_K and Q6_K MUL_MAT and
MUL_MAT_ID sections are kept in ``tiled_ref_kq.bin``, the Q2_K, Q3_K and
IQ4_XS ones in ``tiled_ref_k23x.bin`` and the smallest MUL_MAT section of each
IQ1 / IQ2 / IQ3 type in ``tiled_ref_iq.bin`` (the whole file is 18 MB).  Also one GGUF file of the reference's tokenizer tests
(crates/llama/tests/tokenizer_fixtures/vocab/ggml-vocab-llama-spm.gguf, a
vocab-only model whose metadata vocab.rs:4290-4305 checks) for the GGUF
reader's known-answer test.

Run once in a container where the reference tree is mounted:
    python tests/golden/extract_fixtures.py /root/reference/parity
"""
import os
import shutil
import struct
import sys

WHOLE = [
    "quants_ref.bin", "quants_ref_fp4.bin", "mulmat_ref.bin", "mulmat_ref_c1.bin",
    "q4k_repack_ref.bin", "q4_0_repack_ref.bin", "repack_ref.bin",
    "fa_ref.bin", "fa_probe.bin",
    # real GGUF tensors x the reference's production path (vec_dot.rs:2798-2807)
    "q4k_goss_ref.bin", "q4k_granite_ref.bin", "q6k_granite_ref.bin",
    "q5_0_goss_ref.bin", "q8_0_goss_ref.bin", "q5k_real_ref.bin",
    # IQ4_NL / IQ4_XS quantizer and dequantizer outputs, and the x86 vec_dot
    # results of NVFP4 / IQ4_NL / IQ4_XS (and the other types of that dump)
    # on LCG block bytes and runtime-quantized activations
    "quants_ref_iq.bin", "vecdot3_ref.bin", "quants_ref_q1q2.bin",
]
# row bytes per 256 elements of every type in tiled_ref.bin
ROW_BYTES_PER_256 = {10: 84, 11: 110, 12: 144, 13: 176, 14: 210, 23: 136,
                     16: 66, 17: 74, 22: 82, 18: 98, 21: 110, 19: 50, 29: 56}


def extract_tiled(src, dst, keep=(12, 13, 14), smallest_mm_only=False):
    """VMT1 sections (tiled.rs:2020-2090): kind 0 = MUL_MAT {xq, y, dst},
    kind 1 = MUL_MAT_ID {n_as, n_ids, ne12; xq, y, ids, dst}.
    smallest_mm_only: per kept type, only its smallest MUL_MAT section."""
    b = open(src, "rb").read()
    o = 0
    secs = []
    while True:
        (magic,) = struct.unpack_from("<I", b, o)
        if magic == 0xFFFFFFFF:
            break
        start = o
        o += 4
        kind, ty, n, rows, cols = struct.unpack_from("<5I", b, o)
        o += 20
        rs = (n // 256) * ROW_BYTES_PER_256[ty]
        if kind == 0:
            o += rs * rows + n * cols * 4 + rows * cols * 4
        else:
            n_as, n_ids, ne12 = struct.unpack_from("<3I", b, o)
            o += 12
            o += rs * rows * n_as + n * cols * ne12 * 4 + n_ids * ne12 * 4 + rows * n_ids * ne12 * 4
        if ty in keep:
            secs.append((kind, ty, start, o))
    if smallest_mm_only:
        best = {}
        for kind, ty, a, e in secs:
            if kind == 0 and (ty not in best or e - a < best[ty][1] - best[ty][0]):
                best[ty] = (a, e)
        secs = [(0, ty, a, e) for kind, ty, a, e in secs if kind == 0 and best[ty] == (a, e)]
    out = bytearray()
    for _, _, a, e in secs:
        out += b[a:e]
    out += struct.pack("<I", 0xFFFFFFFF)
    open(dst, "wb").write(bytes(out))


def main(parity_dir):
    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref")
    os.makedirs(here, exist_ok=True)
    for f in WHOLE:
        shutil.copyfile(os.path.join(parity_dir, f), os.path.join(here, f))
    extract_tiled(os.path.join(parity_dir, "tiled_ref.bin"), os.path.join(here, "tiled_ref_kq.bin"))
    # the Q2_K, Q3_K and IQ4_XS sections of the same file, in a file of their own
    extract_tiled(os.path.join(parity_dir, "tiled_ref.bin"), os.path.join(here, "tiled_ref_k23x.bin"), keep=(10, 11, 23))
    # the smallest MUL_MAT section of each IQ1 / IQ2 / IQ3 type
    extract_tiled(os.path.join(parity_dir, "tiled_ref.bin"), os.path.join(here, "tiled_ref_iq.bin"),
                  keep=(16, 17, 18, 19, 21, 22, 29), smallest_mm_only=True)
    vocab = os.path.join(os.path.dirname(parity_dir), "crates", "llama", "tests", "tokenizer_fixtures", "vocab",
                         "ggml-vocab-llama-spm.gguf")
    shutil.copyfile(vocab, os.path.join(here, "ggml-vocab-llama-spm.gguf"))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/parity")
