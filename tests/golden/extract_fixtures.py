"""Copy the reference's committed parity fixtures for the quantized hot path.

The files under ``parity/`` of fly88oj/llama.rust (MIT licence, copyright 2026
fly88oj) are golden vectors that an instrumented llama.cpp build produced.  They
are data (inputs and expected outputs), copied verbatim -- except
``tiled_ref.bin``, of which only the Q4_K / Q6_K MUL_MAT sections are kept (the
other weight types are out of scope and the file is 18 MB).

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
]
ROW_BYTES_PER_256 = {10: 84, 11: 110, 12: 144, 13: 176, 14: 210}


def extract_tiled(src, dst, keep=(12, 14)):
    b = open(src, "rb").read()
    o = 0
    out = bytearray()
    while True:
        (magic,) = struct.unpack_from("<I", b, o)
        if magic == 0xFFFFFFFF:
            break
        start = o
        o += 4
        kind, ty, n, rows, cols = struct.unpack_from("<5I", b, o)
        o += 20
        if kind != 0 or ty not in ROW_BYTES_PER_256:
            break  # the Q2_K..Q6_K mm sections come first; stop at the rest
        o += (n // 256) * ROW_BYTES_PER_256[ty] * rows + n * cols * 4 + rows * cols * 4
        if ty in keep:
            out += b[start:o]
    out += struct.pack("<I", 0xFFFFFFFF)
    open(dst, "wb").write(bytes(out))


def main(parity_dir):
    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref")
    os.makedirs(here, exist_ok=True)
    for f in WHOLE:
        shutil.copyfile(os.path.join(parity_dir, f), os.path.join(here, f))
    extract_tiled(os.path.join(parity_dir, "tiled_ref.bin"), os.path.join(here, "tiled_ref_q4k_q6k.bin"))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/parity")
