"""ghip_mul_mat_noalloc: the same results as ghip_mul_mat on its fixed scratch
(include/ghip.h), with no device allocation by the library."""
import ctypes as C
import gc

import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def noalloc(be, w, wtype, k, x, out):
    import ghip
    L = ghip.lib()
    L.ghip_mul_mat_noalloc.restype = C.c_int
    L.ghip_mul_mat_noalloc.argtypes = [C.c_void_p, C.POINTER(ghip.Tensor), C.POINTER(ghip.Tensor),
                                       C.POINTER(ghip.Tensor), C.c_void_p]
    a, b, d = ghip.describe(w, wtype, k), ghip.describe(x, ghip.F32, k), ghip.describe(out, ghip.F32)
    st = L.ghip_mul_mat_noalloc(be._ctx, C.byref(a), C.byref(b), C.byref(d),
                                C.c_void_p(torch.cuda.current_stream().cuda_stream))
    if st != 0:
        raise ghip.GhipError(f"ghip_mul_mat_noalloc: status {st}: {L.ghip_last_error(be._ctx).decode()}")
    return out


def test_noalloc_matches_mul_mat():
    """Two calls in a row (the second with a smaller input), each bit-equal to
    ghip_mul_mat; device free memory does not change across the calls; a call
    beyond the scratch size is refused with a status."""
    import ghip
    torch.manual_seed(0)
    be = ghip.Backend(0)
    k, n = 4096, 4096
    w4 = be.quantize(torch.randn((n, k), device="cuda") * 0.02, ghip.Q4_K)
    w6 = be.quantize(torch.randn((n, k), device="cuda") * 0.02, ghip.Q6_K)
    cases = [(w4, ghip.Q4_K, 300), (w4, ghip.Q4_K, 20), (w6, ghip.Q6_K, 96), (w6, ghip.Q6_K, 3)]
    xs = [torch.randn((m, k), device="cuda") for _, _, m in cases]
    outs = [torch.full((m, n), float("nan"), device="cuda") for _, _, m in cases]
    # reference results first (these may grow the context's owned workspace)
    want = [be.mul_mat(w, t, k, x).clone() for (w, t, _), x in zip(cases, xs)]
    torch.cuda.synchronize()
    be.close()
    # a fresh context: nothing but the no-allocation entry point runs on it
    be = ghip.Backend(0)
    # no collector run (which could free another test's context) between the
    # two readings of the device's free memory
    gc.collect()
    gc.disable()
    try:
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        for (w, t, _), x, o in zip(cases, xs, outs):
            noalloc(be, w, t, k, x, o)
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
    finally:
        gc.enable()
    for o, ref in zip(outs, want):
        assert torch.equal(o, ref)
    assert free1 == free0
    # the Q6_K prefill GEMM on 14336 -> 4096 at 512 tokens repacks 66 MB of
    # weights into the scratch: refused
    wd = be.quantize(torch.randn((4096, 14336), device="cuda") * 0.02, ghip.Q6_K)
    xd = torch.randn((512, 14336), device="cuda")
    with pytest.raises(ghip.GhipError, match="scratch"):
        noalloc(be, wd, ghip.Q6_K, 14336, xd, torch.empty((512, 4096), device="cuda"))
    # and the array keeps working after the refusal
    o = torch.empty_like(outs[1])
    noalloc(be, w4, ghip.Q4_K, k, xs[1], o)
    torch.cuda.synchronize()
    assert torch.equal(o, want[1])
    be.close()
