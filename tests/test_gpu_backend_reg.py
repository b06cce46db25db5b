"""libggml-hip.so loaded as llama.rust's ggml_backend_load loads it
(crates/ggml/src/backend.rs:1354-1420) on the GPU box: the device list, and a
MUL_MAT driven only through function pointers from get_proc_address, bit-equal
to the same call through ghip.h."""
import ctypes as C

import pytest
import torch

import backend_reg as BR
import ghip

pytestmark = pytest.mark.gpu


def test_load_and_devices():
    print("backend_reg: load + devices", flush=True)
    b = BR.load()
    assert b.api_version == 2 and b.name == "HIP"
    devs = b.devices()
    assert len(devs) >= 1
    d = devs[0]
    assert d.name == "HIP0"
    assert d.type == "gpu"
    assert d.description
    free, total = d.memory
    assert total > 200 * 2**30  # 288 GB of HBM3E
    assert 0 < free <= total


def test_mul_mat_through_proc_addresses():
    print("backend_reg: mul_mat via get_proc_address", flush=True)
    b = BR.load()
    dev = b.devices()[0]
    P = C.POINTER(ghip.Tensor)
    init = C.CFUNCTYPE(C.c_int, C.c_int, C.POINTER(C.c_void_p))(b.proc_address("ghip_init"))
    free = C.CFUNCTYPE(None, C.c_void_p)(b.proc_address("ghip_free"))
    mul_mat = C.CFUNCTYPE(C.c_int, C.c_void_p, P, P, P, C.c_void_p)(b.proc_address("ghip_mul_mat"))
    sync = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_void_p)(b.proc_address("ghip_synchronize"))
    ctx = C.c_void_p()
    assert init(dev.ordinal, C.byref(ctx)) == 0
    try:
        k, n = 4096, 1024
        be = ghip.Backend(0)
        g = torch.Generator(device="cuda").manual_seed(5)
        w = be.quantize(torch.randn((n, k), device="cuda", generator=g) * 0.02, ghip.Q4_K)
        x = torch.randn((3, k), device="cuda", generator=g)
        want = be.mul_mat(w, ghip.Q4_K, k, x)
        out = torch.empty((3, n), dtype=torch.float32, device="cuda")
        a, bb, d = ghip.describe(w, ghip.Q4_K, k), ghip.describe(x, ghip.F32, k), ghip.describe(out, ghip.F32)
        s = torch.cuda.current_stream().cuda_stream
        assert mul_mat(ctx, C.byref(a), C.byref(bb), C.byref(d), s) == 0
        assert sync(ctx, s) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, want)
    finally:
        free(ctx)
