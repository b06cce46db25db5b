"""GPU parity of GGML_OP_MUL_MAT for the further decode weight types Q5_0, Q8_0
(Q8_0 activations) and Q5_K (Q8_K activations), against the CPU oracle and
against the reference's own dumps (mulmat_ref.bin / mulmat_ref_c1.bin,
types 6, 8, 13).

Two kinds of weights:
  * the reference quantizers' output for N(0, 0.02) rows (quantize_row_q5_0_ref,
    quantize_row_q8_0_ref, quantize_row_q5_K_ref) -- the bar: Q8 activation
    bytes and int32 sub-sums bit-exact, fp32 within 1e-5 by
    rel_err = max |a-b| / max(|b|, 1) (vec_dot.rs:2355);
  * random block bytes with finite f16 scales, which reach every code, qh bit
    and packed 6-bit scale: sub-sums bit-exact, fp32 within 1e-4.  Random
    Q5_K mins up to 63 * dmin make the reference's own order (main and min
    terms summed apart, subtracted at the end, vec_dot.rs:940-978) cancel
    terms of ~1e3, so its fp32 result carries ~1e-3 of rounding of its own.
"""
import numpy as np
import pytest

import fixtures as fx
import oracle_lib as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-5
TYPES = [O.Q5_0, O.Q8_0, O.Q5_K]
# Q4_1 / Q5_1: d * q + m weights with Q8_1 activations (vec_dot.rs:620-720);
# no reference dump holds them, the oracle is pinned by quants_ref.bin and a
# brute force (test_oracle_golden.py test_q41_q51_vec_dot_brute_force)
MIN_TYPES = [O.Q4_1, O.Q5_1]
# Q2_K / Q3_K: 2- and 3-bit K-quants with Q8_K activations (vec_dot.rs:758-834);
# the oracle's dequantizers are pinned by quants_ref.bin, its dots by a brute
# force (test_oracle_golden.py test_q2k_q3k_vec_dot_brute_force)
K23_TYPES = [O.Q2_K, O.Q3_K]


@pytest.fixture(scope="module")
def be():
    import ghip
    b = ghip.Backend(0)
    yield b
    b.close()


def rel_err(a, b):
    return float(np.max(np.abs(a - b) / np.maximum(np.abs(b), 1.0))) if a.size else 0.0


def random_blocks(ty, n, rows, seed):
    """rows x n of random `ty` blocks; d (and dmin) are f16 in [2^-10, 2^-4)"""
    rng = np.random.default_rng(seed)
    qk, bs = O.BLOCK[ty]
    w = rng.integers(0, 256, size=(rows, n // qk, bs), dtype=np.uint8)
    offs = {O.Q2_K: (80, 82), O.Q3_K: (108,)}.get(ty, (0, 2) if ty in (O.Q5_K, O.Q4_1, O.Q5_1) else (0,))
    for off in offs:
        e = rng.integers(0x1400, 0x2c00, size=(rows, n // qk), dtype=np.uint16)
        w[:, :, off:off + 2] = e.view(np.uint8).reshape(rows, n // qk, 2)
    return w.reshape(rows, (n // qk) * bs)


def quantized(ty, n, rows, seed):
    if ty in K23_TYPES:
        # no Q2_K / Q3_K quantizer here: the reference's own quantized bytes
        # (quants_ref.bin, 4 super-blocks), rows cycled through its blocks
        q = {tid: q for (_, tid, _n, q, _d) in fx.quant_sections("quants_ref.bin")}[ty].reshape(4, -1)
        nb = n // 256
        idx = (np.arange(rows)[:, None] + np.arange(nb)[None, :] + seed) % 4
        return np.ascontiguousarray(q[idx].reshape(rows, -1))
    wf = (np.random.default_rng(seed).standard_normal((rows, n)) * 0.02).astype(np.float32)
    return O.quantize(ty, wf).reshape(rows, O.row_size(ty, n))


def run_case(be, ty, n, rows, cols, seed=0, check_sub=True, x=None, weights="quant"):
    w = quantized(ty, n, rows, seed) if weights == "quant" else random_blocks(ty, n, rows, seed)
    tol = TOL if weights == "quant" else 1e-4
    if x is None:
        x = np.random.default_rng(seed + 1).standard_normal((cols, n)).astype(np.float32)
    want, route, want_sub = O.mul_mat(ty, w, n, rows, x, cols, want_subsums=check_sub)
    wd = torch.from_numpy(w).cuda()
    xd = torch.from_numpy(x).cuda()
    print(f"case type={ty} n={n} rows={rows} cols={cols} route={route}", flush=True)
    got = be.mul_mat(wd, ty, n, xd).cpu().numpy()
    act = be.mul_mat_act(wd, ty, n, xd).cpu().numpy().reshape(-1)
    assert np.array_equal(act, O.mul_mat_act(ty, n, rows, x, cols)), "activation bytes differ"
    if check_sub:
        sub = be.mul_mat_subsums(wd, ty, n, xd).cpu().numpy()
        assert np.array_equal(sub, want_sub), "int32 sub-sums differ"
    if ty in K23_TYPES and check_sub:
        # the GPU folds d8*d*isum (- d8*dmin*summs) once per super-block: it is
        # held against the float64 value of the exact integer sums (the
        # oracle's export, checked bit-exact above) within gamma_(nb+16) of the
        # terms' magnitudes, and against the fp32 oracle (the reference's 8-lane
        # order, whose own error follows its lane partials) within 1e-4
        nb = n // 256
        wb = w.reshape(rows, nb, -1)
        off = 80 if ty == O.Q2_K else 108
        d = wb[..., off:off + 2].copy().view(np.float16)[..., 0].astype(np.float64)
        act8 = O.mul_mat_act(ty, n, rows, x, cols).reshape(cols, nb, 292)
        d8 = act8[..., 0:4].copy().view(np.float32)[..., 0].astype(np.float64)
        if ty == O.Q2_K:
            dm = wb[..., 82:84].copy().view(np.float16)[..., 0].astype(np.float64)
            t_main = d8[:, None] * d[None] * want_sub[..., 0]
            t_min = d8[:, None] * dm[None] * want_sub[..., 1]
            exact = (t_main - t_min).sum(-1)
            mag = (np.abs(t_main) + np.abs(t_min)).sum(-1)
        else:
            t_main = d8[:, None] * d[None] * want_sub
            exact = t_main.sum(-1)
            mag = np.abs(t_main).sum(-1)
        bound = 2.0 * (nb + 16) * 2.0 ** -24 * mag
        assert np.all(np.abs(got.astype(np.float64) - exact) <= bound), \
            f"max excess {np.max(np.abs(got - exact) - bound):.3e}"
        assert rel_err(got, want) <= 1e-4
        return
    if ty in MIN_TYPES:
        # d * d8 * isum + m * s per block, summed over nb blocks in different
        # orders by the reference (8 lanes + a separate m * s chain) and the
        # kernel: each carries at most gamma_(nb+16) = (nb + 16) * 2^-24 of the
        # sum of the terms' magnitudes (recursive summation bound)
        mag = min_term_magnitudes(ty, w, n, rows, O.mul_mat_act(ty, n, rows, x, cols), cols)
        nb = n // 32
        bound = 2.0 * (nb + 16) * 2.0 ** -24 * mag
        assert np.all(np.abs(got.astype(np.float64) - want) <= bound), \
            f"max excess {np.max(np.abs(got - want) - bound):.3e}"
        assert rel_err(got, want) <= 1e-4
        return
    err = rel_err(got, want)
    assert err <= tol, f"rel_err {err:.3e}"


def min_term_magnitudes(ty, w, n, rows, act, cols):
    """sum_b |d_w d8 isum_b| + |m_w s_b| per output [cols, rows] (float64)."""
    bs = 20 if ty == O.Q4_1 else 24
    b = w.reshape(rows, n // 32, bs)
    d = b[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    m = b[..., 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    qs = b[..., bs - 16:]
    codes = np.concatenate([qs & 15, qs >> 4], axis=-1).astype(np.int64)
    if ty == O.Q5_1:
        qh = b[..., 4:8].copy().view(np.uint32)[..., 0].astype(np.int64)
        codes |= ((qh[..., None] >> np.arange(32)) & 1) << 4
    a = act.reshape(cols, n // 32, 36)
    d8 = a[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    s8 = a[..., 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    q8 = a[..., 4:].view(np.int8).astype(np.int64)
    isum = np.einsum("rbe,cbe->crb", codes, q8)
    return (np.abs(d[None] * d8[:, None] * isum) + np.abs(m[None] * s8[:, None])).sum(-1)


@pytest.mark.parametrize("ty", TYPES + MIN_TYPES)
@pytest.mark.parametrize("cols", [1, 2, 3, 4, 5, 8, 11])
def test_small_shapes(be, ty, cols):
    for n, rows in [(512, 64), (1024, 72), (768, 100), (256, 8)]:
        run_case(be, ty, n, rows, cols, seed=cols + ty)
        run_case(be, ty, n, rows, cols, seed=cols + ty, weights="random")


@pytest.mark.parametrize("ty", TYPES + MIN_TYPES)
def test_ragged_k(be, ty):
    """K not a multiple of one wavefront's span; an odd number of 32-blocks
    (the last lane holds a lone block)"""
    if ty == O.Q5_K:
        run_case(be, ty, 2816, 24, 1)
        run_case(be, ty, 2816, 24, 3, weights="random")
    else:
        run_case(be, ty, 32 * 45, 16, 1)
        run_case(be, ty, 32 * 45, 13, 4, weights="random")
        run_case(be, ty, 2880, 24, 2)


@pytest.mark.parametrize("ty", TYPES + MIN_TYPES)
@pytest.mark.parametrize("n,rows", [(4096, 4096), (14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("cols", [1, 2, 8])
def test_llama_decode_shapes(be, ty, n, rows, cols):
    run_case(be, ty, n, rows, cols, seed=3, check_sub=(cols <= 2))


@pytest.mark.parametrize("name", ["mulmat_ref_c1.bin", "mulmat_ref.bin"])
def test_reference_dumps_on_gpu(be, name):
    """the reference's own outputs (4 rows x 1024, 1 or 3 columns), computed by
    the GPU from the dumped weight bytes and activations"""
    seen = set()
    for tid, n, rows, cols, xq, y, dst in fx.mulmat_sections(name):
        if tid not in TYPES:
            continue
        wd = torch.from_numpy(np.ascontiguousarray(xq).reshape(rows, -1)).cuda()
        xd = torch.from_numpy(np.ascontiguousarray(y, dtype=np.float32).reshape(cols, n)).cuda()
        print(f"dump {name} type={tid}", flush=True)
        got = be.mul_mat(wd, tid, n, xd).cpu().numpy()
        assert rel_err(got, dst) <= TOL, (tid, rel_err(got, dst))
        seen.add(tid)
    assert seen == set(TYPES)


def test_zero_and_extreme_codes(be):
    """all-zero activations, and Q8_0 weights holding -128 (never produced by
    the quantizer, valid for the dot)"""
    n, rows = 1024, 16
    x = np.zeros((2, n), dtype=np.float32)
    x[1] = np.random.default_rng(9).standard_normal(n).astype(np.float32)
    for ty in TYPES + MIN_TYPES:
        run_case(be, ty, n, rows, 2, seed=11, x=x.copy())
        run_case(be, ty, n, rows, 2, seed=11, x=x.copy(), weights="random")
    w = random_blocks(O.Q8_0, n, rows, 12).reshape(rows, n // 32, 34)
    w[:, :, 2:] = 0x80
    w = w.reshape(rows, -1)
    want, _, want_sub = O.mul_mat(O.Q8_0, w, n, rows, x, 2, want_subsums=True)
    got = be.mul_mat(torch.from_numpy(w).cuda(), O.Q8_0, n, torch.from_numpy(x).cuda()).cpu().numpy()
    sub = be.mul_mat_subsums(torch.from_numpy(w).cuda(), O.Q8_0, n, torch.from_numpy(x).cuda()).cpu().numpy()
    assert np.array_equal(sub, want_sub)
    assert rel_err(got, want) <= 1e-4



@pytest.mark.parametrize("ty", K23_TYPES)
@pytest.mark.parametrize("cols", [1, 2, 3, 4, 5, 8, 11])
def test_k23_small_shapes(be, ty, cols):
    """Q2_K / Q3_K: the reference's quantized blocks and random block bytes,
    1-11 columns (launches of at most 4), partial row groups"""
    for n, rows in [(1024, 64), (2048, 72), (256, 8)]:
        run_case(be, ty, n, rows, cols, seed=cols + ty)
        run_case(be, ty, n, rows, cols, seed=cols + ty, weights="random")


@pytest.mark.parametrize("ty", K23_TYPES)
@pytest.mark.parametrize("n,rows,cols", [(4096, 4096, 1), (14336, 4096, 2), (4096, 14336, 4), (2816, 24, 3)])
def test_k23_decode_shapes(be, ty, n, rows, cols):
    """the Llama decode shapes and a K of 11 super-blocks (several wavefronts
    per row, the last one partly empty)"""
    run_case(be, ty, n, rows, cols, seed=5, weights="random")
