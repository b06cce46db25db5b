"""GPU parity of GGML_OP_MUL_MAT with the IQ1 / IQ2 / IQ3 codebook weights
(IQ1_S, IQ1_M, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S; vec_dot.rs:1215-1590,
tiled.rs:440-640) against the CPU oracle.

The oracle is pinned bit-exact on the reference's own dots (vecdot3_ref.bin)
and tiled outputs (tiled_ref_iq.bin) in test_oracle_golden.py.  There is no
quantizer for these formats in the reference, so the weights here are random
block bytes with model-scale d (what a quantized N(0, 0.02) matrix holds) and
the reference's own dumped rows.  Bar: Q8_K activation bytes and the int32
super-block sums bit-exact; fp32 within 1e-5 by rel_err (vec_dot.rs:2355),
or on the reference's dumps the gap between its own two routes.
"""
import numpy as np
import pytest

import fixtures as fx
import oracle_lib as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-5
TYPES = list(O.IQ_GRID_TYPES)


@pytest.fixture(scope="module")
def be():
    import ghip
    b = ghip.Backend(0)
    yield b
    b.close()


def rel_err(a, b):
    return float(np.max(np.abs(a - b) / np.maximum(np.abs(b), 1.0))) if a.size else 0.0


def random_blocks(ty, rows, k, seed):
    """random bytes, the super-block scale d set to model scale (IQ1_M: its
    f16 spread over the top nibbles of the four scale words)"""
    rng = np.random.default_rng(seed)
    bs = O.BLOCK[ty][1]
    nb = k // 256
    b = rng.integers(0, 256, size=(rows, nb, bs), dtype=np.uint8)
    lo, hi = {O.IQ3_S: (2.0 ** -11, 2.0 ** -9)}.get(ty, (2.0 ** -12, 2.0 ** -10))
    d = (rng.uniform(lo, hi, size=(rows, nb)) * rng.choice([-1, 1], size=(rows, nb))).astype(np.float16)
    bits = d.view(np.uint16).astype(np.uint32)
    if ty == O.IQ1_M:
        for m in range(4):  # nibble m of d goes to the top nibble of scale word m
            w = b[..., 48 + 2 * m].astype(np.uint32) | (b[..., 49 + 2 * m].astype(np.uint32) << 8)
            w = (w & 0x0FFF) | (((bits >> (4 * m)) & 0xF) << 12)
            b[..., 48 + 2 * m] = (w & 0xFF).astype(np.uint8)
            b[..., 49 + 2 * m] = (w >> 8).astype(np.uint8)
    else:
        b[..., 0] = (bits & 0xFF).astype(np.uint8)
        b[..., 1] = (bits >> 8).astype(np.uint8)
    return b.reshape(rows, -1)


def check(be, ty, w, k, x, bar=TOL):
    rows, cols = w.shape[0], x.shape[0]
    want, route, want_sub = O.mul_mat(ty, w, k, rows, x, cols, want_subsums=True)
    want = want.reshape(cols, rows)
    wd, xd = torch.from_numpy(np.ascontiguousarray(w)).cuda(), torch.from_numpy(x).cuda()
    print(f"iq type={ty} k={k} rows={rows} cols={cols} route={route}", flush=True)
    got = be.mul_mat(wd, ty, k, xd).cpu().numpy()
    err = rel_err(got, want)
    print(f"  rel_err {err:.2e} (bar {bar:.2e})", flush=True)
    assert err <= bar, (err, bar)
    assert np.array_equal(be.mul_mat_act(wd, ty, k, xd).cpu().numpy().reshape(-1), O.mul_mat_act(ty, k, rows, x, cols))
    sub = be.mul_mat_subsums(wd, ty, k, xd).cpu().numpy()
    assert np.array_equal(sub.reshape(-1), want_sub.reshape(-1))


@pytest.mark.parametrize("ty", TYPES)
@pytest.mark.parametrize("k,rows,cols", [(256, 8, 1), (512, 100, 2), (1024, 37, 3), (4096, 256, 5), (4096, 96, 8),
                                         (2048, 130, 12)])
def test_random_blocks(be, ty, k, rows, cols):
    """decode at 1-5 columns (the row vec_dot) and 8-12 (the reference's tiled
    route; the GPU's fold is the tiled kernel's), rows not a multiple of 8"""
    w = random_blocks(ty, rows, k, seed=k + rows + cols + ty)
    x = np.random.default_rng(cols).standard_normal((cols, k)).astype(np.float32)
    check(be, ty, w, k, x)


@pytest.mark.parametrize("ty", TYPES)
def test_reference_dot(be, ty):
    """the reference's own dot (vecdot3_ref.bin: its x86 kernel on its block
    bytes and quantized activation row), src1 handed over as Q8_K"""
    (sec,) = [s for s in fx.vecdot3_sections() if s[0] == ty]
    _, n, xq, yq, want = sec
    got = be.mul_mat(torch.from_numpy(xq.reshape(1, -1)).cuda(), ty, n,
                     torch.from_numpy(yq.reshape(1, -1)).cuda()).cpu().numpy().reshape(-1)[0]
    assert abs(float(got) - float(want)) <= TOL * max(1.0, abs(float(want))), (got, want)


@pytest.mark.parametrize("ty", TYPES)
def test_reference_tiled_sections(be, ty):
    """the reference's tiled outputs (tiled_ref_iq.bin, random block bytes of
    outputs that cancel): the GPU within 1e-5 or the reference's own
    vec_dot-vs-tiled gap on these inputs, whichever is larger"""
    for tid, n, rows, cols, xq, y, dst in [s for s in fx.tiled_sections("tiled_ref_iq.bin") if s[0] == ty]:
        vd = np.concatenate([O.mul_mat(tid, xq.reshape(rows, -1), n, rows, y[c:c + 1], 1)[0] for c in range(cols)])
        gap = rel_err(vd.reshape(dst.shape), dst)
        print(f"tiled iq type={tid} n={n} rows={rows} cols={cols} gap {gap:.2e}", flush=True)
        got = be.mul_mat(torch.from_numpy(xq.reshape(rows, -1)).cuda(), tid, n,
                         torch.from_numpy(np.ascontiguousarray(y)).cuda()).cpu().numpy()
        assert rel_err(got.reshape(dst.shape), dst) <= max(TOL, gap)
