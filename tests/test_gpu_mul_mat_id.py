"""GPU parity of GGML_OP_MUL_MAT_ID with MXFP4 experts against the CPU oracle.

Bar: the per-block int32 dots bit-exact (checked against a numpy brute force
over the reference's Q8_0 activation bytes) and the fp32 outputs identical to
the oracle's fold (repack.rs:1071-1073 for rows % 8 == 0, compute.rs:7140-7150
otherwise) -- the GPU applies the same operations in the same order, so the
comparison is exact equality, well inside the 1e-5 rel_err bar.
"""
import numpy as np
import pytest

import oracle_lib as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

KV = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], dtype=np.int64)


@pytest.fixture(scope="module")
def be():
    import ghip
    b = ghip.Backend(0)
    yield b
    b.close()


def make(n, rows, n_as, n_tokens, ne11, n_ids, seed=0):
    rng = np.random.default_rng(seed)
    wf = (rng.standard_normal((n_as * rows, n)) * 0.02).astype(np.float32)
    w = O.quantize(O.MXFP4, wf).reshape(n_as, rows, O.row_size(O.MXFP4, n))
    b = rng.standard_normal((n_tokens, ne11, n)).astype(np.float32)
    ids = np.stack([rng.permutation(n_as)[:n_ids] for _ in range(n_tokens)]).astype(np.int32) \
        if n_ids <= n_as else rng.integers(0, n_as, (n_tokens, n_ids)).astype(np.int32)
    return w, b, ids


def brute_dots(w, b, ids, n):
    """int32 block dots sum kvalue(nibble) * q8 from the raw bytes."""
    n_tokens, n_ids = ids.shape
    ne11 = b.shape[1]
    nb = n // 32
    q8 = O.quantize(O.Q8_0, b.reshape(-1, n), kind="quantize_row_q8_0").reshape(n_tokens, ne11, nb, 34)
    qs8 = q8[..., 2:].view(np.int8).astype(np.int64)                      # [t, i11, nb, 32]
    blk = w.reshape(w.shape[0], w.shape[1], nb, 17)
    nib = np.concatenate([blk[..., 1:] & 15, blk[..., 1:] >> 4], axis=-1)  # [e, r, nb, 32]
    kv = KV[nib]
    out = np.zeros((n_tokens, n_ids, w.shape[1], nb), dtype=np.int64)
    for t in range(n_tokens):
        for s in range(n_ids):
            out[t, s] = np.einsum("rbk,bk->rb", kv[ids[t, s]], qs8[t, s % ne11])
    return out.astype(np.int32)


def run(be, n, rows, n_as, n_tokens, ne11, n_ids, seed=0, check_sub=True):
    w, b, ids = make(n, rows, n_as, n_tokens, ne11, n_ids, seed)
    print(f"mul_mat_id n={n} rows={rows} n_as={n_as} tokens={n_tokens} ne11={ne11} n_ids={n_ids}", flush=True)
    want = O.mul_mat_id_mxfp4(w, n, rows, n_as, b, ne11, n_tokens, ids, n_ids)
    wd, bd, idd = (torch.from_numpy(a).cuda() for a in (w, b, ids))
    got = be.mul_mat_id(wd, n, bd, idd).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"max |diff| {np.max(np.abs(got - want)):.3e}"
    if check_sub:
        sub = be.mul_mat_id_subsums(wd, n, bd, idd).cpu().numpy()
        assert np.array_equal(sub, brute_dots(w, b, ids, n)), "int32 block dots differ"


@pytest.mark.parametrize("rows", [64, 40, 20, 7])
@pytest.mark.parametrize("n_tokens,ne11,n_ids", [(1, 1, 4), (3, 2, 2), (37, 1, 4), (20, 4, 4)])
def test_small(be, rows, n_tokens, ne11, n_ids):
    run(be, 96, rows, 6, n_tokens, ne11, n_ids)


def test_skewed_routing(be):
    """Every pair on one expert: many full tiles of one expert plus a tail."""
    n, rows, n_as, n_tokens, n_ids = 64, 136, 4, 150, 1
    w, b, ids = make(n, rows, n_as, n_tokens, 1, n_ids, seed=3)
    ids[:] = 2
    want = O.mul_mat_id_mxfp4(w, n, rows, n_as, b, 1, n_tokens, ids, n_ids)
    got = be.mul_mat_id(*(torch.from_numpy(a).cuda() for a in (w,)), n, torch.from_numpy(b).cuda(),
                        torch.from_numpy(ids).cuda()).cpu().numpy()
    assert np.array_equal(got, want)


def test_large_k_and_tiles(be):
    """K = 2880 (90 blocks: 11 full LDS groups + a 2-block tail), rows past 128, 64-pair tiles."""
    run(be, 2880, 264, 8, 96, 1, 4, seed=4, check_sub=False)
    run(be, 2880, 72, 3, 40, 4, 4, seed=5, check_sub=True)


def test_invalid_ids_give_nan(be):
    n, rows, n_as, n_tokens, n_ids = 64, 16, 4, 5, 2
    w, b, ids = make(n, rows, n_as, n_tokens, 1, n_ids, seed=6)
    bad = ids.copy()
    bad[1, 0] = -1
    bad[3, 1] = n_as
    got = be.mul_mat_id(torch.from_numpy(w).cuda(), n, torch.from_numpy(b).cuda(),
                        torch.from_numpy(bad).cuda()).cpu().numpy()
    want = O.mul_mat_id_mxfp4(w, n, rows, n_as, b, 1, n_tokens, ids, n_ids)
    assert np.all(np.isnan(got[1, 0])) and np.all(np.isnan(got[3, 1]))
    ok = np.ones((n_tokens, n_ids), bool)
    ok[1, 0] = ok[3, 1] = False
    assert np.array_equal(got[ok], want[ok])


def test_empty(be):
    w, b, ids = make(64, 16, 2, 1, 1, 1)
    out = be.mul_mat_id(torch.from_numpy(w).cuda(), 64, torch.zeros((0, 1, 64), device="cuda"),
                        torch.zeros((0, 1), dtype=torch.int32, device="cuda"))
    assert out.shape == (0, 1, 16)


@pytest.mark.parametrize("which", ["gate_up", "down"])
def test_config4(be, which):
    """gpt-oss-shaped: 32 experts, 256 tokens, top-4; gate_up 2880->5760 with
    b broadcast over the slots (ne11 = 1), down 2880->2880 with one b row per
    slot (ne11 = 4).  Weights are quantized on the GPU (pinned separately)."""
    n, n_as, n_tokens, n_ids = 2880, 32, 256, 4
    rows, ne11 = (5760, 1) if which == "gate_up" else (2880, 4)
    g = torch.Generator(device="cuda").manual_seed(11)
    wf = torch.randn((n_as * rows, n), device="cuda", generator=g) * 0.02
    wd = be.quantize(wf, O.MXFP4).view(n_as, rows, -1)
    del wf
    rng = np.random.default_rng(12)
    b = rng.standard_normal((n_tokens, ne11, n)).astype(np.float32)
    logits = rng.standard_normal((n_tokens, n_as))
    ids = np.argsort(-logits, axis=1)[:, :n_ids].astype(np.int32)
    print(f"config4 {which}", flush=True)
    got = be.mul_mat_id(wd, n, torch.from_numpy(b).cuda(), torch.from_numpy(ids).cuda()).cpu().numpy()
    want = O.mul_mat_id_mxfp4(wd.cpu().numpy(), n, rows, n_as, b, ne11, n_tokens, ids, n_ids)
    assert np.array_equal(got, want), f"max |diff| {np.max(np.abs(got - want)):.3e}"
