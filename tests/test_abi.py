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


def _t(ty, ne, nb):
    import sys
    sys.path.insert(0, os.path.join(ROOT, "llama.rust_amd"))
    import ghip
    t = ghip.Tensor()
    t.type, t.ne[:], t.nb[:] = ty, ne, nb
    return t


def test_supports_op_rejects_empty_rows():
    """ne00 == 0 has no decode-kernel geometry: rejected (not a division by zero
    in the host planner)."""
    import ghip
    a = _t(ghip.Q4_K, (0, 64, 1, 1), (144, 0, 0, 0))
    b = _t(ghip.F32, (0, 3, 1, 1), (4, 0, 0, 0))
    d = _t(ghip.F32, (64, 3, 1, 1), (4, 256, 768, 768))
    P = ctypes.POINTER(ghip.Tensor)
    srcs = (P * 2)(ctypes.pointer(a), ctypes.pointer(b))
    assert ghip.lib().ghip_supports_op(ghip.OP_MUL_MAT, ctypes.byref(d), srcs, 2) == 0


def test_supports_op_fa_mask_planes():
    """FLASH_ATTN_EXT takes mask planes broadcast to heads (h % ne2) and to
    sequences (i3 % ne3) when they divide the heads and sequences
    (ggml.c:5517-5518), and sequences (ne3) that q, k, v and dst agree on;
    anything else is refused."""
    import ghip
    D, T, H, S, Hkv = 128, 4, 8, 256, 2
    q = _t(ghip.F32, (D, T, H, 1), (4, 4 * D, 4 * D * T, 4 * D * T * H))
    k = _t(ghip.F16, (D, S, Hkv, 1), (2, 2 * D, 2 * D * S, 2 * D * S * Hkv))
    v = _t(ghip.F16, (D, S, Hkv, 1), (2, 2 * D, 2 * D * S, 2 * D * S * Hkv))
    m = _t(ghip.F16, (S, T, 1, 1), (2, 2 * S, 2 * S * T, 2 * S * T))
    d = _t(ghip.F32, (D, H, T, 1), (4, 4 * D, 4 * D * H, 4 * D * H * T))
    P = ctypes.POINTER(ghip.Tensor)
    srcs = (P * 5)(ctypes.pointer(q), ctypes.pointer(k), ctypes.pointer(v), ctypes.pointer(m), None)
    L = ghip.lib()
    ok = lambda: L.ghip_supports_op(ghip.OP_FLASH_ATTN_EXT, ctypes.byref(d), srcs, 5)
    assert ok() == 1
    m.ne[2], m.nb[3] = H, 2 * S * T * H      # one plane per head
    assert ok() == 1
    m.ne[2] = 3                              # 8 heads % 3 planes != 0
    assert ok() == 0
    m.ne[2] = 2
    for t in (q, k, v, d):                   # two sequences
        t.ne[3] = 2
    assert ok() == 1
    m.ne[3] = 2
    assert ok() == 1
    k.ne[3] = 1                              # k with one sequence, q with two
    assert ok() == 0


def test_workspace_size_query_without_gpu():
    """ghip_workspace_size is host arithmetic: a Q4_K prefill GEMM needs its
    layout (int8 codes, bsum16 as f16, block scales; f32 activations are
    quantized straight into it); a fused decode GEMV needs none."""
    import ghip
    L = ghip.lib()
    P = ctypes.POINTER(ghip.Tensor)

    def need(m):
        a = _t(ghip.Q4_K, (4096, 4096, 1, 1), (144, 2304, 2304 * 4096, 2304 * 4096))
        b = _t(ghip.F32, (4096, m, 1, 1), (4, 16384, 16384 * m, 16384 * m))
        d = _t(ghip.F32, (4096, m, 1, 1), (4, 16384, 16384 * m, 16384 * m))
        srcs = (P * 2)(ctypes.pointer(a), ctypes.pointer(b))
        out = ctypes.c_size_t(7)
        assert L.ghip_workspace_size(ghip.OP_MUL_MAT, ctypes.byref(d), srcs, 2, ctypes.byref(out)) == 0
        return out.value

    assert need(512) >= 512 * 4096 + 16 * 512 * (32 + 4)
    assert need(1) >= 0
