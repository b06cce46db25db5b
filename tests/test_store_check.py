"""Host-side check of every MUL_MAT route's launch windows, without a GPU.

A dry-run context (ghip_init_dry_run) plans each op, takes a workspace
address range and, instead of launching, checks that the byte window every
kernel stores to -- worked out from that launch's own arguments -- lies inside
the buffers the op writes (dst, sub-sums, quantized activations, workspace).
The device pointers below are never dereferenced.  Every route (decode GEMV,
matrix-core decode, split K, the Q4_K / Q6_K / int8 GEMMs, batched planes)
must pass; a deliberately skewed leading dimension (GHIP_DEBUG_LDD_SKEW, a
wrong plan of the kind that once let kernels store past dst) must be caught.
"""
import ctypes as C
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "llama.rust_amd"))

W_BASE, X_BASE, D_BASE, S_BASE = 1 << 40, 2 << 40, 3 << 40, 5 << 40


def _lib():
    import ghip
    L = ghip.lib()
    L.ghip_init_dry_run.restype = C.c_int
    L.ghip_init_dry_run.argtypes = [C.POINTER(C.c_void_p)]
    return ghip, L


def _tensor(ghip, ty, ne, elem_bytes, blck, data):
    t = ghip.Tensor()
    t.type = ty
    ne = list(ne) + [1] * (4 - len(ne))
    t.ne[:] = ne
    nb0 = elem_bytes
    nb1 = ne[0] // blck * elem_bytes
    t.nb[:] = [nb0, nb1, nb1 * ne[1], nb1 * ne[1] * ne[2]]
    t.data = data
    return t


def _run(ty, k, n, m, planes=(1, 1), sub=False):
    ghip, L = _lib()
    ctx = C.c_void_p()
    assert L.ghip_init_dry_run(C.byref(ctx)) == 0
    try:
        blck, bs = ghip.BLOCK[ty]
        a = _tensor(ghip, ty, [k, n, 1, 1], bs, blck, W_BASE)
        b = _tensor(ghip, ghip.F32, [k, m, *planes], 4, 1, X_BASE)
        d = _tensor(ghip, ghip.F32, [n, m, *planes], 4, 1, D_BASE)
        if sub:
            st = L.ghip_mul_mat_subsums(ctx, C.byref(a), C.byref(b), C.c_void_p(S_BASE), None)
        else:
            st = L.ghip_mul_mat(ctx, C.byref(a), C.byref(b), C.byref(d), None)
        return st, L.ghip_last_error(ctx).decode()
    finally:
        L.ghip_free(ctx)


def _types():
    import ghip
    return [ghip.Q4_0, ghip.Q4_1, ghip.Q5_0, ghip.Q5_1, ghip.Q8_0, ghip.Q2_K, ghip.Q3_K, ghip.Q4_K, ghip.Q5_K,
            ghip.Q6_K, ghip.IQ4_NL, ghip.IQ4_XS, ghip.NVFP4, ghip.Q1_0, ghip.Q2_0, ghip.F32, ghip.F16, ghip.BF16,
            ghip.IQ2_XXS, ghip.IQ2_XS, ghip.IQ2_S, ghip.IQ3_XXS, ghip.IQ3_S, ghip.IQ1_S, ghip.IQ1_M]


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 11, 16, 40, 64, 200, 512])
def test_every_route_stores_inside_its_buffers(m):
    import ghip
    for ty in _types():
        for k, n in [(4096, 4096), (4096, 14336), (14336, 4096), (1024, 100)]:
            st, msg = _run(ty, k, n, m)
            assert st == 0, (ty, k, n, m, msg)
            if m <= 8 and ty not in (ghip.F32, ghip.F16, ghip.BF16):
                st, msg = _run(ty, k, n, m, sub=True)
                assert st == 0, ("sub", ty, k, n, m, msg)


def test_batched_planes_store_inside_dst():
    import ghip
    for ty in (ghip.Q4_K, ghip.Q8_0, ghip.Q6_K):
        for m in (1, 5, 64):
            st, msg = _run(ty, 1024, 256, m, planes=(3, 2))
            assert st == 0, (ty, m, msg)


def test_skewed_leading_dimension_is_caught():
    """The same ops with a wrong leading dimension handed to the kernels: the
    check refuses the launch, for the decode, split-K and GEMM routes (from
    two activation rows: one row spans no stride)."""
    code = (
        "import sys; sys.path.insert(0, %r); sys.path.insert(0, %r)\n"
        "import test_store_check as T, ghip\n"
        "for ty, m in [(ghip.Q4_0, 2), (ghip.Q4_K, 2), (ghip.Q4_K, 6), (ghip.Q6_K, 6), (ghip.Q4_K, 64),"
        " (ghip.Q8_0, 64), (ghip.Q6_K, 128)]:\n"
        "    st, msg = T._run(ty, 4096, 4096, m)\n"
        "    assert st != 0 and 'store check' in msg, (ty, m, st, msg)\n"
        "    print(ty, m, msg)\n"
    ) % (os.path.join(ROOT, "tests"), os.path.join(ROOT, "llama.rust_amd"))
    env = dict(os.environ, GHIP_DEBUG_LDD_SKEW="1")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count("store check") == 7


def test_mul_mat_id_stores_inside_dst():
    ghip, L = _lib()
    L.ghip_mul_mat_id.restype = C.c_int
    for ty in [t for t in _types() if t not in (ghip.F32, ghip.F16, ghip.BF16)] + [ghip.MXFP4]:
        for n_tokens, n_ids, ne11 in [(1, 4, 1), (12, 2, 2), (64, 4, 1)]:
            ctx = C.c_void_p()
            assert L.ghip_init_dry_run(C.byref(ctx)) == 0
            try:
                k, rows, n_as = 2048, 96, 8
                blck, bs = ghip.BLOCK[ty]
                a = _tensor(ghip, ty, [k, rows, n_as, 1], bs, blck, W_BASE)
                b = _tensor(ghip, ghip.F32, [k, ne11, n_tokens, 1], 4, 1, X_BASE)
                ids = _tensor(ghip, ghip.I32, [n_ids, n_tokens, 1, 1], 4, 1, S_BASE)
                d = _tensor(ghip, ghip.F32, [rows, n_ids, n_tokens, 1], 4, 1, D_BASE)
                st = L.ghip_mul_mat_id(ctx, C.byref(a), C.byref(b), C.byref(ids), C.byref(d), None)
                assert st == 0, (ty, n_tokens, L.ghip_last_error(ctx).decode())
            finally:
                L.ghip_free(ctx)
