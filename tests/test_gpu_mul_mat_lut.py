"""GPU parity of GGML_OP_MUL_MAT with the table-lookup 4-bit weights IQ4_NL,
IQ4_XS and NVFP4 (vec_dot.rs:1154, :1597, :1655) and the 1- and 2-bit code
weights Q1_0 and Q2_0 (vec_dot.rs:1074, :1120) against the CPU oracle.

The oracle's dots are pinned bit-exact on the reference's x86 results
(parity/vecdot3_ref.bin) and its dequantizers on the reference quantizer's
bytes (quants_ref_iq.bin, quants_ref_fp4.bin, quants_ref_q1q2.bin) in
test_oracle_golden.py.  The weights are (a) the reference quantizer's own
IQ4_NL / IQ4_XS / Q1_0 / Q2_0 rows and (b) random
block bytes with finite scales, as the reference's own vec_dot dump uses.

Bar (north star): activation bytes and int32 sub-sums bit-exact; fp32 outputs
within 1e-5 by rel_err = max |a-b| / max(|b|, 1) (vec_dot.rs:2355).
"""
import numpy as np
import pytest

import fixtures as fx
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


def random_blocks(ty, rows, k, seed, large=False):
    """Random block bytes with finite scales.  Model scale (default): f16 d of
    magnitude 2^-13 .. 2^-10 (IQ4_NL; 2^-17 .. 2^-14 for IQ4_XS, whose group
    scales reach 32) and UE4M3 sub-block scales
    2^-10 .. 2^-7 (NVFP4), so weights are ~0.05 like a quantized N(0, 0.02)
    matrix.  large=True: d up to 2^-6 and UE4M3 up to 2^-4 (weights up to ~2),
    the range of the reference's vec_dot dump."""
    rng = np.random.default_rng(seed)
    qk, bs = O.BLOCK[ty]
    b = rng.integers(0, 256, size=(rows, k // qk, bs), dtype=np.uint8)
    if ty in (O.Q1_0, O.Q2_0):  # weights +-d (Q1_0), -d..2d (Q2_0)
        lo, hi = (2.0 ** -2, 2.0 ** 0) if large else (2.0 ** -8, 2.0 ** -5)
        d = rng.uniform(lo, hi, size=(rows, k // qk)) * rng.choice([-1, 1], size=(rows, k // qk))
        b[:, :, 0:2] = d.astype(np.float16).view(np.uint8).reshape(rows, k // qk, 2)
    elif ty in (O.IQ4_NL, O.IQ4_XS):
        lo, hi = (2.0 ** -9, 2.0 ** -6) if large else (2.0 ** -13, 2.0 ** -10)
        if ty == O.IQ4_XS and not large:  # its 6-bit group scales multiply d by up to 32
            lo, hi = lo / 16, hi / 16
        d = rng.uniform(lo, hi, size=(rows, k // qk)) * rng.choice([-1, 1], size=(rows, k // qk))
        b[:, :, 0:2] = d.astype(np.float16).view(np.uint8).reshape(rows, k // qk, 2)
    else:
        lo, hi = (0x10, 0x38) if large else (0x01, 0x20)
        b[:, :, 0:4] = rng.integers(lo, hi, size=(rows, k // qk, 4), dtype=np.uint8)
    return b.reshape(rows, -1)


def exact(ty, w, k, x):
    """float64 dot of the dequantized weights and the dequantized Q8
    activations the reference forms (every product and sum exact to ~1e-16)"""
    rows, cols = w.shape[0], x.shape[0]
    wd = np.stack([O.dequantize(ty, w[r], k) for r in range(rows)]).astype(np.float64)
    act = O.mul_mat_act(ty, k, rows, x, cols).reshape(cols, -1)
    at = O.ACT_TYPE[ty]
    if at == O.Q8_0:
        ad = np.stack([O.dequantize(O.Q8_0, act[c], k) for c in range(cols)]).astype(np.float64)
    else:  # Q8_K rows: codes * d per super-block
        ad = np.zeros((cols, k))
        for c in range(cols):
            for i in range(k // 256):
                blk = act[c, i * 292:(i + 1) * 292]
                ad[c, i * 256:(i + 1) * 256] = (np.frombuffer(blk[4:260].tobytes(), np.int8).astype(np.float64) *
                                                np.frombuffer(blk[:4].tobytes(), np.float32)[0])
    return ad @ wd.T


def check(be, ty, w, k, x, sub=True, bar=None):
    """bar None: the north star's 1e-5.  bar "reference": the reference's own
    fp32 rounding on these inputs -- the GPU result may differ from the
    reference's by at most twice the reference's distance from the exact
    value (or 1e-5, whichever is larger)."""
    rows, cols = w.shape[0], x.shape[0]
    want, route, want_sub = O.mul_mat(ty, w, k, rows, x, cols, want_subsums=sub)
    want = want.reshape(cols, rows)
    wd, xd = torch.from_numpy(np.ascontiguousarray(w)).cuda(), torch.from_numpy(x).cuda()
    print(f"lut type={ty} k={k} rows={rows} cols={cols} route={route}", flush=True)
    got = be.mul_mat(wd, ty, k, xd).cpu().numpy()
    err = rel_err(got, want)
    tol = TOL
    if bar == "reference":
        tol = max(TOL, 2.0 * rel_err(want, exact(ty, w, k, x)))
        if cols >= 8 and ty == O.IQ4_XS:
            # and the reference's own two routes on these inputs (row vec_dot
            # per column against the tiled kernel), as test_tiled_sections
            vd = np.concatenate([O.mul_mat(ty, w, k, rows, x[c:c + 1], 1)[0] for c in range(cols)])
            tol = max(tol, rel_err(vd.reshape(cols, rows), want))
    print(f"  rel_err {err:.2e} (bar {tol:.2e})", flush=True)
    assert err <= tol, (err, tol)
    act = be.mul_mat_act(wd, ty, k, xd).cpu().numpy().reshape(-1)
    assert np.array_equal(act, O.mul_mat_act(ty, k, rows, x, cols))
    if sub:
        s = be.mul_mat_subsums(wd, ty, k, xd).cpu().numpy()
        assert np.array_equal(s.reshape(-1), want_sub.reshape(-1))
    return err


ALL = [O.IQ4_NL, O.IQ4_XS, O.NVFP4, O.Q1_0, O.Q2_0]


@pytest.mark.parametrize("ty", ALL)
@pytest.mark.parametrize("k,rows,cols", [(256, 8, 1), (512, 100, 2), (1024, 37, 3), (4096, 256, 5), (4096, 96, 8),
                                         (2048, 130, 40), (4096, 512, 64)])
def test_random_blocks(be, ty, k, rows, cols):
    """Decode (1..8 rows: the lookup kernels), prefill (32+ rows: the int8
    GEMM for IQ4_NL / IQ4_XS, the decode kernel in groups of 8 columns for
    NVFP4), the int8 GEMM for Q1_0 / Q2_0 too, rows not a multiple of 8, K from one block to 4096; model-scale
    weights, the 1e-5 bar."""
    w = random_blocks(ty, rows, k, seed=k + rows + cols)
    x = np.random.default_rng(cols).standard_normal((cols, k)).astype(np.float32)
    check(be, ty, w, k, x, sub=rows * cols <= 512 * 64)


@pytest.mark.parametrize("ty", ALL)
@pytest.mark.parametrize("k,rows,cols", [(512, 100, 2), (4096, 96, 8), (2048, 130, 40)])
def test_large_random_blocks(be, ty, k, rows, cols):
    """Weights up to ~2 whose outputs cancel (hundreds of units summing to
    near zero): here the reference's own fp32 order already sits ~1e-5 from
    the exact result, so the bar is twice that distance, or for IQ4_XS from 8
    columns the gap between the reference's own vec_dot and tiled routes if
    that is larger."""
    w = random_blocks(ty, rows, k, seed=k + rows + cols, large=True)
    x = np.random.default_rng(cols).standard_normal((cols, k)).astype(np.float32)
    check(be, ty, w, k, x, bar="reference")


@pytest.mark.parametrize("ty", [O.IQ4_NL, O.IQ4_XS, O.Q1_0, O.Q2_0])
def test_reference_quantized_rows(be, ty):
    """The reference quantizer's IQ4_NL / IQ4_XS / Q1_0 / Q2_0 bytes
    (quants_ref_iq.bin, quants_ref_q1q2.bin, one 1024-element row) as a weight
    row, at 1, 5 and 40 activation rows."""
    name = "quants_ref_q1q2.bin" if ty in (O.Q1_0, O.Q2_0) else "quants_ref_iq.bin"
    (sec,) = [s for s in fx.quant_sections(name) if s[1] == ty]
    _, _, n, q, _ = sec
    w = np.tile(q.reshape(1, -1), (16, 1))
    for cols in (1, 5, 40):
        x = np.random.default_rng(cols).standard_normal((cols, n)).astype(np.float32)
        check(be, ty, w, n, x)


@pytest.mark.parametrize("ty", ALL)
def test_reference_dot(be, ty):
    """The reference's own dot (vecdot3_ref.bin: its x86 kernel on its block
    bytes and its quantized activation row), with that activation row handed
    over already quantized (src1 in the vec_dot type), to the matmul bar."""
    import ghip
    (sec,) = [s for s in fx.vecdot3_sections() if s[0] == ty]
    _, n, xq, yq, want = sec
    wd = torch.from_numpy(xq.reshape(1, -1)).cuda()
    yd = torch.from_numpy(yq.reshape(1, -1)).cuda()
    got = be.mul_mat(wd, ty, n, yd).cpu().numpy().reshape(-1)[0]
    assert abs(float(got) - float(want)) <= TOL * max(1.0, abs(float(want))), (got, want)


@pytest.mark.parametrize("ty", [O.IQ4_NL, O.IQ4_XS, O.Q1_0, O.Q2_0])
def test_registered_weight_gemm(be, ty):
    """A registered IQ4_NL / IQ4_XS / Q1_0 / Q2_0 weight keeps its int8-code copy; the GEMM on
    it gives the bits of the per-call repack."""
    import ghip
    k, rows, cols = 1024, 192, 48
    w = random_blocks(ty, rows, k, seed=5)  # model scale
    x = np.random.default_rng(6).standard_normal((cols, k)).astype(np.float32)
    wd, xd = torch.from_numpy(w).cuda(), torch.from_numpy(x).cuda()
    before = be.mul_mat(wd, ty, k, xd).clone()
    be.register_weight(wd, ty, k)
    after = be.mul_mat(wd, ty, k, xd)
    torch.cuda.synchronize()
    be.unregister_weight(wd, ty, k)
    assert torch.equal(before, after)
    want, _, _ = O.mul_mat(ty, w, k, rows, x, cols)
    assert rel_err(after.cpu().numpy(), want.reshape(cols, rows)) <= TOL
