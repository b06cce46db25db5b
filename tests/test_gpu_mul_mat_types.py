"""GPU parity of GGML_OP_MUL_MAT for the further decode weight types Q5_0, Q8_0
(Q8_0 activations), Q4_1 / Q5_1 (Q8_1) and Q5_K / Q2_K / Q3_K (Q8_K), against the CPU oracle and
against the reference's own dumps (mulmat_ref.bin / mulmat_ref_c1.bin,
types 6, 8, 13).

Two kinds of weights:
  * the reference quantizers' output for N(0, 0.02) rows (quantize_row_q5_0_ref,
    quantize_row_q8_0_ref, quantize_row_q5_K_ref) -- the bar: Q8 activation
    bytes and int32 sub-sums bit-exact, fp32 within 1e-5 by
    rel_err = max |a-b| / max(|b|, 1) (vec_dot.rs:2355);
  * random block bytes with finite f16 scales, which reach every code, qh bit
    and packed 6-bit scale: sub-sums bit-exact, fp32 within 1e-5, or within
    twice the distance of the reference's own fp32 result from the exact value
    of its per-block formula where that is larger (random Q5_K / Q2_K mins up
    to 63 * dmin make the reference's order -- main and min terms summed apart,
    subtracted at the end, vec_dot.rs:940-978 -- cancel terms of ~1e3).
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
    if x is None:
        x = np.random.default_rng(seed + 1).standard_normal((cols, n)).astype(np.float32)
    want, route, want_sub = O.mul_mat(ty, w, n, rows, x, cols, want_subsums=True)
    wd = torch.from_numpy(w).cuda()
    xd = torch.from_numpy(x).cuda()
    print(f"case type={ty} n={n} rows={rows} cols={cols} route={route}", flush=True)
    got = be.mul_mat(wd, ty, n, xd).cpu().numpy()
    act = be.mul_mat_act(wd, ty, n, xd).cpu().numpy().reshape(-1)
    assert np.array_equal(act, O.mul_mat_act(ty, n, rows, x, cols)), "activation bytes differ"
    if check_sub:
        sub = be.mul_mat_subsums(wd, ty, n, xd).cpu().numpy()
        assert np.array_equal(sub, want_sub), "int32 sub-sums differ"
    err = rel_err(got, want)
    # held to the bar unless the reference's own fp32 order already sits
    # further from the exact value of its formula (the float64 sum of the
    # exact integer sub-sums, checked bit-exact against the GPU's where
    # check_sub, times their scales): then to twice that distance.  (Q4_1 /
    # Q5_1 at K = 14336 on quantized N(0, 0.02) rows: the reference is
    # 1.0e-5 / 1.2e-5 from that value, its main and m*s sums cancelling.)
    exact, mag = exact_from_subsums(ty, w, n, rows, O.mul_mat_act(ty, n, rows, x, cols), cols, want_sub)
    # every fp32 evaluation order of the formula lies within the recursive
    # summation bound gamma_(nb+16) of the terms' magnitudes of that value
    nb = n // O.BLOCK[ty][0]
    bound = 2.0 * (nb + 16) * 2.0 ** -24 * mag
    assert np.all(np.abs(got.astype(np.float64) - exact) <= bound), \
        f"max excess {np.max(np.abs(got - exact) - bound):.3e}"
    bar = max(TOL, 2.0 * rel_err(want.astype(np.float64), exact))
    if weights == "random":
        # random block bytes (mins up to 63 * dmin against main terms of the
        # same size): where the cancellation makes that bound wider than the
        # bar, two valid orders may differ by it
        bar = max(bar, float(np.max(bound / np.maximum(np.abs(want), 1.0))))
    assert err <= bar, f"rel_err {err:.3e} (bar {bar:.3e})"


def _f16(a, off):
    return a[..., off:off + 2].copy().view(np.float16)[..., 0].astype(np.float64)


def exact_from_subsums(ty, w, n, rows, act, cols, sub):
    """float64 value of the reference's per-block formula from the exact
    integer sub-sums, and the sum of its terms' magnitudes, both [cols, rows]:
    Q5_0 / Q8_0  sum_b d d8 isum_b;  Q4_1 / Q5_1  sum_b d d8 isum_b + m s8_b;
    Q5_K / Q2_K  sum_b d8 (d isum_b - dmin imin_b);  Q3_K  sum_b d8 d isum_b."""
    qk, bs = O.BLOCK[ty]
    nb = n // qk
    wb = w.reshape(rows, nb, bs)
    at = O.ACT_TYPE[ty]
    a = act.reshape(cols, nb, -1)
    if at == O.Q8_K:
        d8 = a[..., 0:4].copy().view(np.float32)[..., 0].astype(np.float64)
    else:
        d8 = _f16(a, 0)
    sub = sub.reshape(cols, rows, nb, -1).astype(np.float64)
    if ty in (O.Q5_0, O.Q8_0):
        t = [_f16(wb, 0)[None] * d8[:, None] * sub[..., 0]]
    elif ty in MIN_TYPES:
        t = [_f16(wb, 0)[None] * d8[:, None] * sub[..., 0], _f16(wb, 2)[None] * _f16(a, 2)[:, None]]
    elif ty in (O.Q5_K, O.Q2_K):
        dd, dm = (_f16(wb, 0), _f16(wb, 2)) if ty == O.Q5_K else (_f16(wb, 80), _f16(wb, 82))
        t = [d8[:, None] * dd[None] * sub[..., 0], -(d8[:, None] * dm[None] * sub[..., 1])]
    else:
        t = [d8[:, None] * _f16(wb, 108)[None] * sub[..., 0]]
    exact = sum(x.sum(-1) for x in t)
    mag = sum(np.abs(x).sum(-1) for x in t)
    return exact, mag


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
    exact, _ = exact_from_subsums(O.Q8_0, w, n, rows, O.mul_mat_act(O.Q8_0, n, rows, x, 2), 2, want_sub)
    assert rel_err(got, want) <= max(TOL, 2.0 * rel_err(want.astype(np.float64), exact))


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
