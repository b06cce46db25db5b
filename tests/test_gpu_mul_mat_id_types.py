"""GPU parity of GGML_OP_MUL_MAT_ID with the further expert types (Q4_0,
Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, IQ4_NL, IQ4_XS, NVFP4, Q1_0, Q2_0).

The reference (compute.rs:1917-2202) quantizes every src1 row to the type's
vec_dot_type, then per (token, slot) pair runs the expert's row vec_dot --
the Q4_0 8x8 repack gemv for experts with rows % 8 == 0 -- except that an
expert of a tiled type (Q2_K, Q3_K, IQ4_XS) with >= 8 routed pairs takes the
tiled kernel over those pairs.  The oracle here follows that: per pair its
one-column MUL_MAT of the expert (whose route is the repack gemv or the row
vec_dot), and for tiled-type experts with >= 8 pairs its MUL_MAT over all of
the expert's pairs at once (the tiled route).  Bar: the integer sub-sums
bit-exact; fp32 within 1e-5 on quantized weights, or the gap between the
reference's own two routes on these inputs where that is larger.
"""
import numpy as np
import pytest

import oracle_lib as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TILED = (O.Q2_K, O.Q3_K, O.IQ4_XS) + tuple(O.IQ_GRID_TYPES)


@pytest.fixture(scope="module")
def be():
    import ghip
    b = ghip.Backend(0)
    yield b
    b.close()


def rel_err(got, want):
    return float(np.max(np.abs(got - want) / np.maximum(np.abs(want), 1.0))) if want.size else 0.0


def weights(ty, n_as, rows, n, rng):
    """the reference's quantizer where the oracle has it, else model-scale
    random blocks (f16 scales of a quantized N(0, 0.02) matrix)"""
    if ty in O.IQ_GRID_TYPES:
        import test_gpu_mul_mat_iq as IQ
        return IQ.random_blocks(ty, n_as * rows, n, int(rng.integers(1 << 30))).reshape(n_as, rows, -1)
    if ty in (O.Q2_K, O.Q3_K, O.IQ4_NL, O.IQ4_XS, O.NVFP4):
        qk, bs = O.BLOCK[ty]
        b = rng.integers(0, 256, size=(n_as * rows, n // qk, bs), dtype=np.uint8)
        def f16(lo, hi, size):
            return (rng.uniform(lo, hi, size=size) * rng.choice([-1, 1], size=size)).astype(np.float16).view(np.uint8)
        shp = (n_as * rows, n // qk)
        if ty == O.Q2_K:
            b[..., 80:82] = f16(2 ** -12, 2 ** -9, shp).reshape(*shp, 2)
            b[..., 82:84] = np.abs(f16(2 ** -13, 2 ** -10, shp).reshape(*shp, 2).view(np.float16)).view(np.uint8)
        elif ty == O.Q3_K:
            b[..., 108:110] = f16(2 ** -13, 2 ** -10, shp).reshape(*shp, 2)
        elif ty == O.IQ4_NL:
            b[..., 0:2] = f16(2 ** -13, 2 ** -10, shp).reshape(*shp, 2)
        elif ty == O.IQ4_XS:
            b[..., 0:2] = f16(2 ** -17, 2 ** -14, shp).reshape(*shp, 2)
        else:
            b[..., 0:4] = rng.integers(0x01, 0x20, size=(*shp, 4), dtype=np.uint8)
        return b.reshape(n_as, rows, -1)
    wf = (rng.standard_normal((n_as * rows, n)) * 0.02).astype(np.float32)
    return O.quantize(ty, wf).reshape(n_as, rows, O.row_size(ty, n))


def oracle_mmid(ty, w, n, rows, ne11, y, ids):
    """(reference route result, per-pair vec_dot result, sub-sums)"""
    n_tokens, n_ids = ids.shape
    per = n // O.BLOCK[ty][0] * {O.Q2_K: 2, O.NVFP4: 4, O.Q1_0: 4, O.Q2_0: 2}.get(ty, 1)
    vd = np.zeros((n_tokens, n_ids, rows), dtype=np.float32)
    sub = np.zeros((n_tokens, n_ids, rows, per), dtype=np.int32)
    for t in range(n_tokens):
        for s in range(n_ids):
            out, _, sb = O.mul_mat(ty, w[ids[t, s]], n, rows, y[t, s % ne11][None], 1, want_subsums=True)
            vd[t, s] = out[0]
            sub[t, s] = sb.reshape(rows, per)
    ref = vd.copy()
    if ty in TILED:
        for e in range(w.shape[0]):
            pairs = [(t, s) for t in range(n_tokens) for s in range(n_ids) if ids[t, s] == e]
            if len(pairs) >= 8:
                x = np.stack([y[t, s % ne11] for t, s in pairs])
                out, route, _ = O.mul_mat(ty, w[e], n, rows, x, len(pairs))
                out = out.reshape(len(pairs), rows)
                for i, (t, s) in enumerate(pairs):
                    ref[t, s] = out[i]
    return ref, vd, sub


TYPES = [O.Q4_0, O.Q4_1, O.Q5_0, O.Q5_1, O.Q8_0, O.Q2_K, O.Q3_K, O.IQ4_NL, O.IQ4_XS, O.NVFP4, O.Q1_0, O.Q2_0] + list(O.IQ_GRID_TYPES)


@pytest.mark.parametrize("ty", TYPES)
@pytest.mark.parametrize("n,rows,n_as,n_tokens,ne11,n_ids", [
    (1024, 64, 4, 1, 1, 4),      # decode: one token, four experts (Q4_0 rows % 8 == 0: the repack gemv)
    (512, 37, 3, 12, 1, 2),      # rows % 8 != 0; some experts with >= 8 pairs (tiled types: tiled route)
    (2048, 24, 5, 9, 2, 2),      # ne11 = n_ids (down-projection shape)
])
def test_further_expert_types(be, ty, n, rows, n_as, n_tokens, ne11, n_ids):
    print(f"mmid type {ty} n={n} rows={rows} n_as={n_as} tokens={n_tokens} ne11={ne11} n_ids={n_ids}", flush=True)
    rng = np.random.default_rng(n + rows + ty)
    w = weights(ty, n_as, rows, n, rng)
    y = rng.standard_normal((n_tokens, ne11, n)).astype(np.float32)
    ids = np.stack([rng.permutation(n_as)[:n_ids] for _ in range(n_tokens)]).astype(np.int32)
    want, vd, want_sub = oracle_mmid(ty, w, n, rows, ne11, y, ids)
    wd, yd, idd = torch.from_numpy(np.ascontiguousarray(w)).cuda(), torch.from_numpy(y).cuda(), torch.from_numpy(ids).cuda()
    got = be.mul_mat_id(wd, n, yd, idd, ty=ty).cpu().numpy()
    bar = max(1e-5, rel_err(vd, want))
    err = rel_err(got, want)
    print(f"  rel_err {err:.2e} (bar {bar:.2e})", flush=True)
    assert err <= bar, (err, bar)
    sub = be.mul_mat_id_subsums(wd, n, yd, idd, ty=ty).cpu().numpy()
    assert np.array_equal(sub.reshape(want_sub.shape), want_sub)


def test_invalid_ids_give_nan_rows(be):
    n, rows, n_as = 256, 16, 2
    rng = np.random.default_rng(1)
    w = weights(O.Q8_0, n_as, rows, n, rng)
    y = rng.standard_normal((2, 1, n)).astype(np.float32)
    ids = np.array([[0, 5], [1, -1]], dtype=np.int32)
    got = be.mul_mat_id(torch.from_numpy(w).cuda(), n, torch.from_numpy(y).cuda(), torch.from_numpy(ids).cuda(),
                        ty=O.Q8_0).cpu().numpy()
    assert np.all(np.isnan(got[0, 1])) and np.all(np.isnan(got[1, 1]))
    want, _, _ = oracle_mmid(O.Q8_0, w, n, rows, 1, y, np.array([[0, 0], [1, 1]], dtype=np.int32))
    assert rel_err(got[0, 0], want[0, 0]) <= 1e-5 and rel_err(got[1, 0], want[1, 0]) <= 1e-5
