"""GPU parity of GGML_OP_MUL_MAT_ID with Q4_K, Q5_K and Q6_K experts.

The reference routes K-quant experts three ways (compute.rs:1917-2202): the
Q4_K 8x8 repack gemv when an expert has rows % 8 == 0, the tiled kernel for
experts with >= 8 routed pairs, the row vec_dot for the rest -- all on
quantize_row_q8_K activations.  The GPU runs one kernel for all of them.
Bar: the per-super-block int32 sums bit-exact against the oracle's (they do
not depend on the route); fp32 outputs within 1e-5 relative of the oracle's
routed result on quantized real-valued weights, and within the rounding bound
the reference's own routes meet on its random-byte fixtures (tiled.rs:2205).
"""
import numpy as np
import pytest

import fixtures as fx
import oracle_lib as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def be():
    import ghip
    b = ghip.Backend(0)
    yield b
    b.close()


def rel_err(got, want):
    return float(np.max(np.abs(got - want) / np.maximum(np.abs(want), 1.0)))


def oracle_mmid(ty, w, n, rows, ne11, y, ids, subsums=False):
    """Every routed pair through the oracle's MUL_MAT of its expert on its
    activation row (route: the reference's for that matrix at one column)."""
    n_tokens, n_ids = ids.shape
    dst = np.zeros((n_tokens, n_ids, rows), dtype=np.float32)
    sub = None
    for t in range(n_tokens):
        for s in range(n_ids):
            out, _, sb = O.mul_mat(ty, w[ids[t, s]], n, rows, y[t, s % ne11][None], 1, want_subsums=subsums)
            dst[t, s] = out[0]
            if subsums:
                if sub is None:
                    sub = np.zeros((n_tokens, n_ids) + sb.shape[1:], dtype=np.int32)
                sub[t, s] = sb[0]
    return dst, sub


def exact_mmid(ty, w, n, rows, ne11, y, ids):
    """The routed products in float64 from the oracle's exact integer
    super-block sums and the block scales (the value every fp32 route rounds),
    and the sum of the magnitudes of their per-block terms (what an fp32
    route's rounding error scales with)."""
    n_tokens, n_ids = ids.shape
    nb = n // 256
    _, sub = oracle_mmid(ty, w, n, rows, ne11, y, ids, subsums=True)
    act = O.mul_mat_act(ty, n, 1, y.reshape(-1, n), n_tokens * ne11).reshape(n_tokens, ne11, nb, 292)
    d8 = act[..., :4].copy().view(np.float32)[..., 0].astype(np.float64)      # block_q8_K.d
    blk = w.reshape(w.shape[0], rows, nb, -1)
    if ty == O.Q6_K:
        dw = blk[..., 208:210].copy().view(np.float16)[..., 0].astype(np.float64)
    else:
        dw = blk[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
        dmin = blk[..., 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    out = np.zeros((n_tokens, n_ids, rows))
    mag = np.zeros((n_tokens, n_ids, rows))
    for t in range(n_tokens):
        for s in range(n_ids):
            e, a = ids[t, s], d8[t, s % ne11]
            if ty == O.Q6_K:
                v = dw[e] * sub[t, s].reshape(rows, nb)
                m = np.abs(v)
            else:
                sb = sub[t, s].reshape(rows, nb, 2).astype(np.float64)
                v = dw[e] * sb[..., 0] - dmin[e] * sb[..., 1]
                m = np.abs(dw[e] * sb[..., 0]) + np.abs(dmin[e] * sb[..., 1])
            out[t, s] = (v * a).sum(axis=1)
            mag[t, s] = (m * np.abs(a)).sum(axis=1)
    return out, mag


@pytest.mark.parametrize("tid", [O.Q4_K, O.Q5_K, O.Q6_K])
def test_reference_mmid_sections(be, tid):
    """The reference's own MUL_MAT_ID vectors (tiled.rs:2118-2189: 140 rows,
    5 experts, 16 tokens).  Their weights are random block bytes, so outputs
    reach ~7e3 from per-block terms that cancel, and each fp32 route rounds
    its own way: the stored dst (tiled kernel) and the reference's per-pair
    row vec_dot differ from the exact value by up to 1e-3 in rel_err.  Bars:
    the integer super-block sums bit-exact against the oracle's; the error
    against the exact value (float64 over those sums) at most 128 units of
    fp32 rounding of the summed term magnitudes -- a bound both reference
    routes meet on these inputs (their worst is 93, Q6_K vec_dot) -- and
    within 1e-6 of dst normwise."""
    u = 2.0 ** -24
    secs = [s for s in fx.tiled_sections(kind=1) if s[0] == tid]
    assert len(secs) == 1
    _, n, rows, ne11, n_as, n_ids, ne12, xq, y, ids, dst = secs[0]
    print(f"mmid fixture type {tid} n={n} rows={rows} n_as={n_as} n_ids={n_ids} tokens={ne12} ne11={ne11}", flush=True)
    wd, yd, idd = torch.from_numpy(xq).cuda(), torch.from_numpy(y).cuda(), torch.from_numpy(ids).cuda()
    got = be.mul_mat_id(wd, n, yd, idd, ty=tid).cpu().numpy()
    args = (tid, xq.reshape(n_as, rows, -1), n, rows, ne11, y.reshape(ne12, ne11, n), ids.reshape(ne12, n_ids))
    vec_dot, want_sub = oracle_mmid(*args, subsums=True)
    exact, mag = exact_mmid(*args)
    vec_dot, exact, mag = (a.reshape(dst.shape) for a in (vec_dot, exact, mag))
    units = lambda x: float(np.max(np.abs(x - exact) / (u * mag)))
    print(f"  rounding units vs exact: gpu {units(got):.1f}, dst {units(dst):.1f}, vec_dot {units(vec_dot):.1f}; "
          f"rel_err gpu vs dst {rel_err(got, dst):.2e}", flush=True)
    assert max(units(dst), units(vec_dot)) <= 128
    assert units(got) <= 128
    assert np.linalg.norm(got - dst) <= 1e-6 * np.linalg.norm(dst)
    sub = be.mul_mat_id_subsums(wd, n, yd, idd, ty=tid).cpu().numpy()
    assert np.array_equal(sub, want_sub.reshape(sub.shape))


@pytest.mark.parametrize("tid,n,rows,n_as,n_tokens,ne11,n_ids", [
    (O.Q4_K, 512, 64, 8, 12, 1, 2),     # rows % 8 == 0: the repack gemv route
    (O.Q4_K, 256, 40, 3, 9, 2, 2),      # rows % 8 == 0, ne11 = n_ids (down-projection shape)
    (O.Q4_K, 768, 37, 6, 20, 1, 3),     # rows % 8 != 0: tiled / vec_dot
    (O.Q5_K, 512, 24, 4, 10, 1, 2),
    (O.Q6_K, 768, 48, 5, 11, 1, 4),
    (O.Q6_K, 256, 21, 2, 17, 2, 2),
    (O.Q4_K, 4608, 16, 4, 5, 1, 2),     # K wider than one wavefront pass (18 super-blocks)
])
def test_random_experts(be, tid, n, rows, n_as, n_tokens, ne11, n_ids):
    print(f"mmid type {tid} n={n} rows={rows} n_as={n_as} tokens={n_tokens} ne11={ne11} n_ids={n_ids}", flush=True)
    rng = np.random.default_rng(n + rows + tid)
    wf = (rng.standard_normal((n_as * rows, n)) * 0.02).astype(np.float32)
    w = O.quantize(tid, wf).reshape(n_as, rows, O.row_size(tid, n))
    y = rng.standard_normal((n_tokens, ne11, n)).astype(np.float32)
    ids = np.stack([rng.permutation(n_as)[:n_ids] for _ in range(n_tokens)]).astype(np.int32)
    want, want_sub = oracle_mmid(tid, w, n, rows, ne11, y, ids, subsums=True)
    wd, yd, idd = torch.from_numpy(w).cuda(), torch.from_numpy(y).cuda(), torch.from_numpy(ids).cuda()
    got = be.mul_mat_id(wd, n, yd, idd, ty=tid).cpu().numpy()
    assert rel_err(got, want) <= 1e-5
    sub = be.mul_mat_id_subsums(wd, n, yd, idd, ty=tid).cpu().numpy()
    assert np.array_equal(sub, want_sub.reshape(sub.shape))


def test_invalid_id_gives_nan(be):
    rng = np.random.default_rng(5)
    n, rows, n_as = 256, 16, 2
    w = O.quantize(O.Q4_K, (rng.standard_normal((n_as * rows, n)) * 0.02).astype(np.float32))
    w = w.reshape(n_as, rows, -1)
    y = rng.standard_normal((3, 1, n)).astype(np.float32)
    ids = np.array([[0], [7], [1]], dtype=np.int32)
    got = be.mul_mat_id(torch.from_numpy(w).cuda(), n, torch.from_numpy(y).cuda(), torch.from_numpy(ids).cuda(),
                        ty=O.Q4_K).cpu().numpy()
    assert np.isnan(got[1]).all() and np.isfinite(got[0]).all() and np.isfinite(got[2]).all()
