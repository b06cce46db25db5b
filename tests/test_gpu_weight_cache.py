"""The device weight cache (ghip_weight_register; the reference's repack
cache, repack.rs:4250-4480) and the Q6_K prefill GEMM's exactness on
extreme valid blocks.

Bar: a registered weight gives bit-identical MUL_MAT results to the per-call
repack, before and after unregistering, also inside a captured HIP graph;
the cache counts what it built (repack_stats, repack.rs:4329) so a second
registration or call is shown to reuse the copy.  The Q6_K GEMM keeps one
fp32 accumulator per scale plane, whose sums are exact integers for any
valid block: on blocks at the extremes (scales -128 / 127, q = 0 / 63,
activations +-127) its super-block sums equal the oracle's int32 ones and
its outputs stay within 1e-5.
"""
import numpy as np
import pytest

import oracle_lib as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def be():
    import ghip
    b = ghip.Backend(0)
    yield b
    b.close()


def rel_err(a, b):
    return float(np.max(np.abs(a - b) / np.maximum(np.abs(b), 1.0))) if a.size else 0.0


def q6k_weights(rows, n, seed):
    rng = np.random.default_rng(seed)
    wf = (rng.standard_normal((rows, n)) * 0.02).astype(np.float32)
    return O.quantize(O.Q6_K, wf).reshape(rows, O.row_size(O.Q6_K, n))


def test_register_reuses_copy_bit_identical(be):
    rows, n, tokens = 256, 1024, 96   # 96 activation rows: the Q6_K GEMM route
    w = torch.from_numpy(q6k_weights(rows, n, 1)).cuda()
    x = torch.from_numpy(np.random.default_rng(2).standard_normal((tokens, n), dtype=np.float32)).cuda()
    print(f"weight cache Q6_K rows={rows} n={n} tokens={tokens}", flush=True)
    before = be.mul_mat(w, O.Q6_K, n, x).clone()
    n0, b0, built0 = be.weight_cache_stats()
    be.register_weight(w, O.Q6_K, n)
    be.register_weight(w, O.Q6_K, n)  # second registration: a hit
    n1, b1, built1 = be.weight_cache_stats()
    assert (n1, built1) == (n0 + 1, built0 + 1)
    assert b1 - b0 == rows * (n // 256) * 336  # one 336-byte GEMM record per super-block
    first = be.mul_mat(w, O.Q6_K, n, x).clone()
    second = be.mul_mat(w, O.Q6_K, n, x).clone()
    assert be.weight_cache_stats()[2] == built1  # calls read the copy, build nothing
    assert torch.equal(first, before) and torch.equal(second, before)
    want, _, _ = O.mul_mat(O.Q6_K, w.cpu().numpy(), n, rows, x.cpu().numpy(), tokens)
    assert rel_err(first.cpu().numpy(), want) <= 1e-5
    be.unregister_weight(w, O.Q6_K, n)
    assert be.weight_cache_stats()[:2] == (n0, b0)
    assert torch.equal(be.mul_mat(w, O.Q6_K, n, x), before)


def test_registered_weight_in_captured_graph(be):
    rows, n, tokens = 128, 512, 64
    w = torch.from_numpy(q6k_weights(rows, n, 3)).cuda()
    x = torch.from_numpy(np.random.default_rng(4).standard_normal((tokens, n), dtype=np.float32)).cuda()
    print(f"weight cache graph Q6_K rows={rows} n={n} tokens={tokens}", flush=True)
    be.register_weight(w, O.Q6_K, n)
    out = torch.empty((tokens, rows), dtype=torch.float32, device="cuda")
    be.mul_mat(w, O.Q6_K, n, x, out=out)  # grows the workspace outside capture
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            be.mul_mat(w, O.Q6_K, n, x, out=out)
    for _ in range(3):
        out.fill_(0.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    be.unregister_weight(w, O.Q6_K, n)


def test_budget_and_other_types(be, monkeypatch):
    """LLAMA_RUST_REPACK_MAX_MB=0: nothing kept (calls repack per call, as
    the reference falls back); LLAMA_RUST_REPACK=0 likewise; a Q4_K weight is
    read in its GGUF layout, so registering it keeps nothing."""
    rows, n = 64, 512
    w = torch.from_numpy(q6k_weights(rows, n, 5)).cuda()
    base = be.weight_cache_stats()
    monkeypatch.setenv("LLAMA_RUST_REPACK_MAX_MB", "0")
    be.register_weight(w, O.Q6_K, n)
    assert be.weight_cache_stats() == base
    monkeypatch.delenv("LLAMA_RUST_REPACK_MAX_MB")
    monkeypatch.setenv("LLAMA_RUST_REPACK", "0")
    be.register_weight(w, O.Q6_K, n)
    assert be.weight_cache_stats() == base
    monkeypatch.delenv("LLAMA_RUST_REPACK")
    wq = torch.from_numpy(O.quantize(O.Q4_K, np.zeros((rows, n), np.float32)).reshape(rows, -1)).cuda()
    be.register_weight(wq, O.Q4_K, n)
    assert be.weight_cache_stats() == base


def extreme_q6k(rows, n, seed):
    """Valid Q6_K blocks at the extremes: per row a pattern of q = 0 / 63 /
    random, scales -128 / 127 / random sign, d = 2^-10."""
    rng = np.random.default_rng(seed)
    nb = n // 256
    blk = np.zeros((rows, nb, 210), dtype=np.uint8)
    for r in range(rows):
        kind = r % 4
        if kind == 0:      # q = 0, sc = -128: every product (-32)(-128)(q8) the same sign
            ql, qh, sc = 0x00, 0x00, np.full(16, -128)
        elif kind == 1:    # q = 63, sc = 127
            ql, qh, sc = 0xFF, 0xFF, np.full(16, 127)
        elif kind == 2:    # q = 0 / 63 by element, scales -128 / 127 by sub-block
            ql, qh, sc = None, None, rng.choice([-128, 127], 16)
        else:              # random bytes, extreme scales
            ql, qh, sc = None, None, rng.choice([-128, 127, -127, 126], 16)
        for b in range(nb):
            blk[r, b, :128] = rng.integers(0, 256, 128) if ql is None else ql
            blk[r, b, 128:192] = rng.integers(0, 256, 64) if qh is None else qh
            blk[r, b, 192:208] = sc.astype(np.int8).view(np.uint8)
            blk[r, b, 208:210] = np.array([2.0 ** -10], dtype=np.float16).view(np.uint8)
    return blk.reshape(rows, nb * 210)


def test_q6K_gemm_extreme_blocks_exact(be):
    rows, n, tokens = 64, 1024, 80
    w = extreme_q6k(rows, n, 11)
    rng = np.random.default_rng(12)
    x = rng.choice([-1.0, 1.0], (tokens, n)).astype(np.float32)
    x[0] = 1.0    # all codes +127 with aligned signs: |is| up to 1.33e8 per super-block
    x[1] = -1.0
    print(f"q6_K GEMM extreme blocks rows={rows} n={n} tokens={tokens}", flush=True)
    want, _, want_sub = O.mul_mat(O.Q6_K, w, n, rows, x, tokens, want_subsums=True)
    assert np.abs(want_sub).max() > 2 ** 24   # the case the per-plane accumulators exist for
    wd, xd = torch.from_numpy(w).cuda(), torch.from_numpy(x).cuda()
    got = be.mul_mat(wd, O.Q6_K, n, xd).cpu().numpy()
    assert rel_err(got, want) <= 1e-5, rel_err(got, want)
    sub = be.mul_mat_subsums(wd, O.Q6_K, n, xd).cpu().numpy()
    assert np.array_equal(sub, want_sub)


@pytest.mark.parametrize("n,rows,n_as,n_tok,n_ids", [
    (2880, 264, 8, 40, 4),   # 90 blocks: 22 whole groups + a 2-block group; rows past 128 (and % 8 == 0)
    (256, 100, 4, 24, 2),    # 8 blocks; rows % 8 != 0: the plain fold; one partial row block
])
def test_register_mxfp4_experts_bit_identical(be, monkeypatch, n, rows, n_as, n_tok, n_ids):
    """Registered MXFP4 experts (the windows laid out in the kernel's staging
    order) give the same bits as the GGUF layout, and the sub-sums agree."""
    import ghip
    monkeypatch.setenv("GHIP_MOE_REG_MIN_ROWS", "0")  # the registered copy at any row count
    rng = np.random.default_rng(rows)
    wf = torch.from_numpy((rng.standard_normal((n_as * rows, n)) * 0.02).astype(np.float32)).cuda()
    w = be.quantize(wf, ghip.MXFP4).view(n_as, rows, -1)
    b = torch.from_numpy(rng.standard_normal((n_tok, 1, n)).astype(np.float32)).cuda()
    ids = torch.from_numpy(np.stack([rng.permutation(n_as)[:n_ids] for _ in range(n_tok)]).astype(np.int32)).cuda()
    print(f"mxfp4 registered n={n} rows={rows} n_as={n_as} tokens={n_tok}", flush=True)
    before = be.mul_mat_id(w, n, b, ids).clone()
    sub0 = be.mul_mat_id_subsums(w, n, b, ids).clone()
    n0, b0, built0 = be.weight_cache_stats()
    be.register_weight(w, ghip.MXFP4, n)
    n1, b1, built1 = be.weight_cache_stats()
    assert (n1, built1) == (n0 + 1, built0 + 1)
    assert b1 - b0 == n_as * ((rows + 127) // 128) * ((n // 32 + 3) // 4) * 128 * 80
    after = be.mul_mat_id(w, n, b, ids)
    assert torch.equal(after.view(torch.int32), before.view(torch.int32))
    sub1 = be.mul_mat_id_subsums(w, n, b, ids)
    assert torch.equal(sub1, sub0)
    be.unregister_weight(w, ghip.MXFP4, n)
    assert be.weight_cache_stats()[:2] == (n0, b0)
