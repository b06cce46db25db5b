"""GPU parity of GGML_OP_MUL_MAT with F32, F16 and BF16 weights against the
CPU oracle (oracle_mul_mat_dense: compute.rs:1680-1745, vec_dot.rs:1700-1727).

The activations are rounded to the weight type as the reference rounds them
(f16 / bf16 round to nearest even), so every product is the same exact value
on both sides; only the fp32 summation order differs.  Bar: 1e-5 by
rel_err = max |a-b| / max(|b|, 1) (vec_dot.rs:2355).
"""
import numpy as np
import pytest

import oracle_lib as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-5


@pytest.fixture(scope="module")
def be():
    import ghip
    b = ghip.Backend(0)
    yield b
    b.close()


def rel_err(a, b):
    return float(np.max(np.abs(a - b) / np.maximum(np.abs(b), 1.0))) if a.size else 0.0


def make(ty, rows, k, seed, scale=0.02):
    rng = np.random.default_rng(seed)
    wf = (rng.standard_normal((rows, k)) * scale).astype(np.float32)
    if ty == O.F32:
        return torch.from_numpy(wf), wf
    if ty == O.F16:
        t = torch.from_numpy(wf).to(torch.float16)
    else:
        t = torch.from_numpy(wf).to(torch.bfloat16)
    return t, t.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("ty", [O.F32, O.F16, O.BF16])
@pytest.mark.parametrize("k,rows,cols", [(4096, 64, 1), (4096, 100, 3), (1000, 37, 8), (14336, 48, 2),
                                         (4096, 256, 11), (77, 9, 5), (128, 4096, 4)])
def test_dense_weights(be, ty, k, rows, cols):
    wt, wbits = make(ty, rows, k, k + rows + cols)
    x = np.random.default_rng(cols).standard_normal((cols, k)).astype(np.float32)
    want = O.mul_mat_dense(ty, wbits, k, rows, x, cols)
    print(f"dense type={ty} k={k} rows={rows} cols={cols}", flush=True)
    got = be.mul_mat(wt.cuda(), ty, k, torch.from_numpy(x).cuda()).cpu().numpy()
    assert rel_err(got, want) <= TOL, rel_err(got, want)


@pytest.mark.parametrize("ty", [O.F16, O.BF16])
def test_activation_rounding_is_the_references(be, ty):
    """activations that differ only below the weight type's precision (ties
    included) give the reference's rounding: exact outputs on unit weights"""
    k, rows = 256, 8
    w = np.zeros((rows, k), dtype=np.float32)
    w[np.arange(rows), np.arange(rows)] = 1.0
    wt = torch.from_numpy(w).to(torch.float16 if ty == O.F16 else torch.bfloat16)
    wbits = wt.view(torch.int16).numpy().view(np.uint16)
    base = np.float32(1.0)
    ulp = 2.0 ** -10 if ty == O.F16 else 2.0 ** -7
    x = np.zeros((1, k), dtype=np.float32)
    x[0, :rows] = base + np.array([0.5, 1.5, 0.25, 0.75, 2.5, -0.5, 0.49, 0.51], dtype=np.float32) * np.float32(ulp)
    want = O.mul_mat_dense(ty, wbits, k, rows, x, 1)
    got = be.mul_mat(wt.cuda(), ty, k, torch.from_numpy(x).cuda()).cpu().numpy()
    assert np.array_equal(got, want)


def test_dense_batched_planes(be):
    """F16 weights with broadcast planes (ne12 = 2 * ne02), as an FA-off KQ"""
    import ghip
    k, rows, m = 128, 64, 5
    w = torch.randn(2, rows, k, generator=torch.Generator().manual_seed(1)).to(torch.float16)
    x = torch.randn(4, m, k, generator=torch.Generator().manual_seed(2))
    import ctypes as C
    out = torch.empty(4, m, rows, device="cuda")
    wd, xd = w.cuda(), x.cuda()
    a, b, d = ghip.describe(wd, ghip.F16), ghip.describe(xd, ghip.F32), ghip.describe(out, ghip.F32)
    st = ghip.lib().ghip_mul_mat(be._ctx, C.byref(a), C.byref(b), C.byref(d), None)
    assert st == 0, ghip.lib().ghip_last_error(be._ctx)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    wb = w.view(torch.int16).numpy().view(np.uint16)
    for p in range(4):
        want = O.mul_mat_dense(O.F16, wb[p // 2], k, rows, x[p].numpy(), m)
        assert rel_err(got[p], want) <= TOL
