"""The C-ABI library loads and exports every entry point include/ghip.h declares
(CPU only: no compute call is made)."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    src = open(os.path.join(ROOT, "include", "ghip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(ghip_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_entry_points():
    names = declared()
    for must in ("ghip_init", "ghip_free", "ghip_mul_mat", "ghip_supports_op"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(os.path.join(ROOT, "llama.rust_amd", "libghip.so"))
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_code_objects_present():
    for k in ("ghip_quant", "ghip_gemv", "ghip_wquant", "ghip_gemm", "ghip_fa", "ghip_moe"):
        assert os.path.exists(os.path.join(ROOT, "llama.rust_amd", k + ".hsaco")), k


def test_supports_op_without_gpu():
    """supports_op is pure host logic (no device call)."""
    import sys
    sys.path.insert(0, os.path.join(ROOT, "llama.rust_amd"))
    import ghip
    L = ghip.lib()
    a, b, d = ghip.Tensor(), ghip.Tensor(), ghip.Tensor()
    a.type, a.ne[:] = ghip.Q4_K, (4096, 64, 1, 1)
    a.nb[:] = (144, 2304, 2304 * 64, 2304 * 64)
    b.type, b.ne[:] = ghip.F32, (4096, 3, 1, 1)
    b.nb[:] = (4, 16384, 16384 * 3, 16384 * 3)
    d.type, d.ne[:] = ghip.F32, (64, 3, 1, 1)
    d.nb[:] = (4, 256, 768, 768)
    P = ctypes.POINTER(ghip.Tensor)
    srcs = (P * 2)(ctypes.pointer(a), ctypes.pointer(b))
    assert L.ghip_supports_op(ghip.OP_MUL_MAT, ctypes.byref(d), srcs, 2) == 1
    b.type = ghip.F16
    assert L.ghip_supports_op(ghip.OP_MUL_MAT, ctypes.byref(d), srcs, 2) == 0
