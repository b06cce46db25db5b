"""ctypes binding of the test-only CPU oracle (oracle/liboracle.so).

Test infrastructure: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg only.
"""
import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
LIB_PATH = os.path.join(ORACLE_DIR, "liboracle.so")

F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K, MXFP4 = 0, 1, 2, 6, 8, 12, 13, 14, 15, 39
Q4_1, Q5_1, Q8_1 = 3, 7, 9
Q2_K, Q3_K = 10, 11
IQ4_NL, IQ4_XS, NVFP4 = 20, 23, 40
Q1_0, Q2_0 = 41, 42
BF16 = 30
IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ3_S, IQ2_S, IQ1_M = 16, 17, 18, 19, 21, 22, 29
IQ_GRID_TYPES = (IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M)
BLOCK = {Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176),
         Q6_K: (256, 210), Q8_K: (256, 292), MXFP4: (32, 17), Q4_1: (32, 20), Q5_1: (32, 24), Q8_1: (32, 36),
         Q2_K: (256, 84), Q3_K: (256, 110), IQ4_NL: (32, 18), IQ4_XS: (256, 136), NVFP4: (64, 36),
         Q1_0: (128, 18), Q2_0: (64, 18), IQ2_XXS: (256, 66), IQ2_XS: (256, 74), IQ2_S: (256, 82),
         IQ3_XXS: (256, 98), IQ3_S: (256, 110), IQ1_S: (256, 50), IQ1_M: (256, 56)}
# weight type -> activation type of its dot (vec_dot_type)
ACT_TYPE = {Q4_0: Q8_0, Q5_0: Q8_0, Q8_0: Q8_0, Q4_K: Q8_K, Q5_K: Q8_K, Q6_K: Q8_K, Q4_1: Q8_1, Q5_1: Q8_1,
            Q2_K: Q8_K, Q3_K: Q8_K, IQ4_NL: Q8_0, IQ4_XS: Q8_K, NVFP4: Q8_0, Q1_0: Q8_0, Q2_0: Q8_0,
            **{t: Q8_K for t in IQ_GRID_TYPES}}
# int32 sub-sums per weight row and activation row (ghip_mul_mat_subsums layout)
def subsums_per_row(ty, n):
    return {Q4_0: n // 32, Q5_0: n // 32, Q8_0: n // 32, Q4_K: (n // 256) * 2, Q5_K: (n // 256) * 2,
            Q6_K: n // 256, Q4_1: n // 32, Q5_1: n // 32, Q2_K: (n // 256) * 2, Q3_K: n // 256,
            IQ4_NL: n // 32, IQ4_XS: n // 256, NVFP4: n // 16, Q1_0: n // 32, Q2_0: n // 32,
            **{t: n // 256 for t in IQ_GRID_TYPES}}[ty]
ROUTE_REPACK, ROUTE_TILED, ROUTE_VECDOT = 1, 2, 3


def row_size(ty, n):
    qk, sz = BLOCK[ty]
    assert n % qk == 0
    return n // qk * sz


def build():
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


class FaArgs(C.Structure):
    _fields_ = [("q", C.c_void_p), ("q_nb1", C.c_int64), ("q_nb2", C.c_int64),
                ("k", C.c_void_p), ("v", C.c_void_p),
                ("k_nb1", C.c_int64), ("k_nb2", C.c_int64), ("v_nb1", C.c_int64), ("v_nb2", C.c_int64),
                ("kv_f16", C.c_int), ("mask", C.c_void_p), ("mask_nb1", C.c_int64),
                ("sinks", C.c_void_p), ("dst", C.c_void_p),
                ("DK", C.c_int), ("DV", C.c_int), ("T", C.c_int), ("H", C.c_int), ("S", C.c_int),
                ("H_kv", C.c_int), ("scale", C.c_float), ("max_bias", C.c_float), ("softcap", C.c_float),
                ("n_chunks", C.c_int), ("nthreads", C.c_int)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, i64, fp = C.c_void_p, C.c_int64, C.POINTER(C.c_float)
        L.oracle_fp32_to_fp16.restype = C.c_uint16
        L.oracle_fp32_to_fp16.argtypes = [C.c_float]
        L.oracle_fp16_to_fp32.restype = C.c_float
        L.oracle_fp16_to_fp32.argtypes = [C.c_uint16]
        L.oracle_nearest_int.restype = C.c_int32
        L.oracle_nearest_int.argtypes = [C.c_float]
        L.oracle_e8m0_to_fp32_half.restype = C.c_float
        L.oracle_e8m0_to_fp32_half.argtypes = [C.c_uint8]
        L.oracle_ue4m3_to_fp32.restype = C.c_float
        L.oracle_ue4m3_to_fp32.argtypes = [C.c_uint8]
        for f in ["quantize_row_q4_0_ref", "quantize_row_q4_K_ref", "quantize_row_q6_K_ref",
                  "quantize_row_q5_0_ref", "quantize_row_q5_K_ref",
                  "quantize_row_mxfp4_ref", "quantize_row_q8_0_ref", "quantize_row_q8_0",
                  "quantize_row_q8_K_ref", "quantize_row_q8_K_mat",
                  "quantize_row_q4_1_ref", "quantize_row_q5_1_ref", "quantize_row_q8_1",
                  "quantize_row_q1_0_ref", "quantize_row_q2_0_ref"]:
            fn = getattr(L, "oracle_" + f)
            fn.restype = None
            fn.argtypes = [vp, vp, i64]
        L.oracle_dequantize_row.restype = None
        L.oracle_dequantize_row.argtypes = [C.c_int, vp, vp, i64]
        for f in ["vec_dot_q4_0_q8_0", "vec_dot_q4_K_q8_K", "vec_dot_q6_K_q8_K", "vec_dot_q5_0_q8_0",
                  "vec_dot_q8_0_q8_0", "vec_dot_q5_K_q8_K", "vec_dot_q4_1_q8_1", "vec_dot_q5_1_q8_1",
                  "vec_dot_q2_K_q8_K", "vec_dot_q3_K_q8_K", "vec_dot_iq4_nl_q8_0", "vec_dot_iq4_xs_q8_K",
                  "vec_dot_nvfp4_q8_0", "vec_dot_q1_0_q8_0", "vec_dot_q2_0_q8_0"]:
            fn = getattr(L, "oracle_" + f)
            fn.restype = C.c_float
            fn.argtypes = [C.c_int, vp, vp]
        L.oracle_mul_mat.restype = C.c_int
        L.oracle_mul_mat.argtypes = [C.c_int, vp, i64, i64, vp, i64, vp, vp, vp, C.c_int]
        L.oracle_mul_mat_act.restype = C.c_int
        L.oracle_mul_mat_act.argtypes = [C.c_int, i64, i64, vp, i64, vp]
        L.oracle_vec_dot_iq.restype = C.c_float
        L.oracle_vec_dot_iq.argtypes = [C.c_int, C.c_int, vp, vp]
        L.oracle_mul_mat_dense.restype = C.c_int
        L.oracle_mul_mat_dense.argtypes = [C.c_int, vp, i64, i64, vp, i64, vp, C.c_int]
        L.oracle_fp32_to_bf16.restype = C.c_uint16
        L.oracle_fp32_to_bf16.argtypes = [C.c_float]
        L.oracle_mul_mat_id_mxfp4.restype = C.c_int
        L.oracle_mul_mat_id_mxfp4.argtypes = [vp, i64, i64, i64, vp, i64, i64, vp, i64, vp, C.c_int]
        L.oracle_flash_attn_ext.restype = C.c_int
        L.oracle_flash_attn_ext.argtypes = [C.POINTER(FaArgs)]
        L.oracle_wtime.restype = C.c_double
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


_QUANT = {Q4_0: "quantize_row_q4_0_ref", Q4_K: "quantize_row_q4_K_ref",
          Q6_K: "quantize_row_q6_K_ref", MXFP4: "quantize_row_mxfp4_ref",
          Q5_0: "quantize_row_q5_0_ref", Q5_K: "quantize_row_q5_K_ref", Q8_0: "quantize_row_q8_0_ref",
          Q4_1: "quantize_row_q4_1_ref", Q5_1: "quantize_row_q5_1_ref", Q8_1: "quantize_row_q8_1",
          Q1_0: "quantize_row_q1_0_ref", Q2_0: "quantize_row_q2_0_ref"}


def quantize(ty, x, kind=None):
    """Quantize rows of x (f32, last dim = row length) with the reference quantizer."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1]
    rows = x.size // n
    name = kind or _QUANT[ty]
    out_ty = {"quantize_row_q8_0_ref": Q8_0, "quantize_row_q8_0": Q8_0,
              "quantize_row_q8_K_ref": Q8_K, "quantize_row_q8_K_mat": Q8_K,
              "quantize_row_q8_1": Q8_1}.get(name, ty)
    out = np.zeros(rows * row_size(out_ty, n), dtype=np.uint8)
    getattr(lib(), "oracle_" + name)(_p(x), _p(out), x.size)
    return out


def dequantize(ty, q, k):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    out = np.zeros(k, dtype=np.float32)
    lib().oracle_dequantize_row(ty, _p(q), _p(out), k)
    return out


def mul_mat(ty, w, n, rows, x, cols, want_subsums=False, nthreads=0):
    """Routed MUL_MAT: returns (out [cols, rows] f32, route, subsums or None)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size == n * cols
    out = np.zeros((cols, rows), dtype=np.float32)
    sub = None
    if want_subsums:
        sub = np.zeros((cols, rows, subsums_per_row(ty, n)), dtype=np.int32)
    route = C.c_int(0)
    rc = lib().oracle_mul_mat(ty, _p(np.ascontiguousarray(w)), n, rows, _p(x), cols, _p(out),
                              _p(sub), C.byref(route), nthreads)
    if rc < 0:
        raise ValueError(f"oracle_mul_mat rc={rc}")
    if sub is not None and ty in (Q4_K, Q5_K, Q2_K):
        sub = sub.reshape(cols, rows, n // 256, 2)
    return out, route.value, sub


def mul_mat_act(ty, n, rows, x, cols):
    x = np.ascontiguousarray(x, dtype=np.float32)
    act_ty = ACT_TYPE[ty]
    act = np.zeros(cols * row_size(act_ty, n), dtype=np.uint8)
    rc = lib().oracle_mul_mat_act(ty, n, rows, _p(x), cols, _p(act))
    if rc < 0:
        raise ValueError(f"oracle_mul_mat_act rc={rc}")
    return act


def vec_dot_iq(ty, n, xq, yq):
    """the row dot of an IQ1 / IQ2 / IQ3 row with a Q8_K row (vec_dot.rs:1215-1590)"""
    return np.float32(lib().oracle_vec_dot_iq(ty, n, _p(np.ascontiguousarray(xq)), _p(np.ascontiguousarray(yq))))


def mul_mat_dense(ty, w, n, rows, x, cols, nthreads=0):
    """F32 / F16 / BF16 weights (w: rows x n as float32 or uint16 bits) -> out [cols, rows]"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros((cols, rows), dtype=np.float32)
    rc = lib().oracle_mul_mat_dense(ty, _p(np.ascontiguousarray(w)), n, rows, _p(x), cols, _p(out), nthreads)
    if rc < 0:
        raise ValueError(f"oracle_mul_mat_dense rc={rc}")
    return out


def fp32_to_bf16(f):
    return lib().oracle_fp32_to_bf16(float(f))


def mul_mat_id_mxfp4(as_q, n, rows, n_as, b, ne11, n_tokens, ids, n_ids, nthreads=0):
    b = np.ascontiguousarray(b, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    dst = np.zeros((n_tokens, n_ids, rows), dtype=np.float32)
    rc = lib().oracle_mul_mat_id_mxfp4(_p(np.ascontiguousarray(as_q)), n, rows, n_as, _p(b), ne11,
                                       n_tokens, _p(ids), n_ids, _p(dst), nthreads)
    if rc < 0:
        raise ValueError(f"oracle_mul_mat_id_mxfp4 rc={rc}")
    return dst


def wtime():
    return lib().oracle_wtime()


def flash_attn_ext(q, k, v, mask=None, sinks=None, scale=1.0, max_bias=0.0, softcap=0.0, n_chunks=1,
                   nthreads=0):
    """q [H, T, DK] f32, k [H_kv, S, DK], v [H_kv, S, DV] (float16 or float32),
    mask [T, S] float16 or None, sinks [H] f32 or None.
    Returns (dst [T, H, DV] f32, path)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    kv_f16 = k.dtype == np.float16
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v, dtype=k.dtype)
    H, T, DK = q.shape
    H_kv, S, _ = k.shape
    DV = v.shape[2]
    dst = np.zeros((T, H, DV), dtype=np.float32)
    a = FaArgs()
    a.q, a.q_nb1, a.q_nb2 = q.ctypes.data, DK, T * DK
    a.k, a.v = k.ctypes.data, v.ctypes.data
    a.k_nb1, a.k_nb2, a.v_nb1, a.v_nb2 = DK, S * DK, DV, S * DV
    a.kv_f16 = int(kv_f16)
    if mask is not None:
        mask = np.ascontiguousarray(mask, dtype=np.float16)
        a.mask, a.mask_nb1 = mask.ctypes.data, mask.shape[1]
    if sinks is not None:
        sinks = np.ascontiguousarray(sinks, dtype=np.float32)
        a.sinks = sinks.ctypes.data
    a.dst = dst.ctypes.data
    a.DK, a.DV, a.T, a.H, a.S, a.H_kv = DK, DV, T, H, S, H_kv
    a.scale, a.max_bias, a.softcap = scale, max_bias, softcap
    a.n_chunks = n_chunks
    a.nthreads = nthreads or (os.cpu_count() or 1)
    path = lib().oracle_flash_attn_ext(C.byref(a))
    if path < 0:
        raise ValueError("oracle_flash_attn_ext: bad shape")
    return dst, path
