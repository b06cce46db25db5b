"""GPU parity of GGML_OP_MUL_MAT (Q4_0 / Q4_K / Q6_K) against the CPU oracle.

Bar: Q8 activation bytes and int32 sub-sums bit-exact;
fp32 outputs within 1e-5 of the reference path by the reference's own
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


def make(ty, n, rows, cols, seed=0, scale=0.02):
    rng = np.random.default_rng(seed)
    wf = (rng.standard_normal((rows, n)) * scale).astype(np.float32)
    w = O.quantize(ty, wf).reshape(rows, O.row_size(ty, n))
    x = np.random.default_rng(seed + 1).standard_normal((cols, n)).astype(np.float32)
    return w, x


def run_case(be, ty, n, rows, cols, seed=0, x=None, check_sub=True, w=None):
    w0, x0 = make(ty, n, rows, cols, seed)
    if x is None:
        x = x0
    if w is None:
        w = w0
    if ty == O.Q4_0 and rows % 8 and cols >= 2:
        # the reference's tinyBLAS route (llamafile_sgemm), absent from the
        # oracle: the same Q8_0 rows and integer block dots, checked against
        # the row vec_dot per column (the fp32 order is all that differs)
        per = [O.mul_mat(ty, w, n, rows, x[c:c + 1], 1, want_subsums=check_sub) for c in range(cols)]
        want = np.concatenate([p[0] for p in per])
        want_sub = np.concatenate([p[2] for p in per]) if check_sub else None
        want_act = np.concatenate([O.mul_mat_act(ty, n, rows, x[c:c + 1], 1) for c in range(cols)])
        route = "tinyBLAS (checked per column against vec_dot)"
    else:
        want, route, want_sub = O.mul_mat(ty, w, n, rows, x, cols, want_subsums=check_sub)
        want_act = O.mul_mat_act(ty, n, rows, x, cols)
    wd = torch.from_numpy(w).cuda()
    xd = torch.from_numpy(x).cuda()
    print(f"case type={ty} n={n} rows={rows} cols={cols} route={route}", flush=True)
    got = be.mul_mat(wd, ty, n, xd).cpu().numpy()
    act = be.mul_mat_act(wd, ty, n, xd).cpu().numpy().reshape(-1)
    assert np.array_equal(act, want_act), "activation bytes differ"
    if check_sub:
        sub = be.mul_mat_subsums(wd, ty, n, xd).cpu().numpy()
        assert np.array_equal(sub, want_sub), "int32 sub-sums differ"
    err = rel_err(got, want)
    assert err <= TOL, f"rel_err {err:.3e}"
    return err


@pytest.mark.parametrize("ty", [O.Q4_0, O.Q4_K, O.Q6_K])
@pytest.mark.parametrize("cols", [1, 2, 3, 4, 5, 8, 11])
def test_small_shapes(be, ty, cols):
    for n, rows in [(512, 64), (1024, 72), (768, 100), (256, 8)]:
        run_case(be, ty, n, rows, cols, seed=cols)


@pytest.mark.parametrize("ty", [O.Q4_0, O.Q4_K, O.Q6_K])
def test_ragged_k(be, ty):
    # K not a multiple of one wavefront's span; odd number of Q4_0 blocks
    n = 2880 if ty == O.Q4_0 else 2816
    if ty == O.Q4_0:
        run_case(be, ty, 32 * 45, 16, 1)
    run_case(be, ty, n, 24, 1)
    run_case(be, ty, n, 24, 4)


def test_q8K_edge_rows(be):
    """Zero rows, ties of |max| with opposite signs, and a value whose scaled
    product lands exactly on .5 -- the quantizer branches of quants.rs:615-650
    and repack.rs:1561-1620."""
    n, rows = 512, 16
    w, _ = make(O.Q4_K, n, rows, 6)
    x = np.random.default_rng(5).standard_normal((6, n)).astype(np.float32)
    x[0] = 0.0
    x[1, :] = 0.25
    x[1, 7] = -3.0
    x[1, 100] = 3.0
    x[2, 3] = x[2].max() + 1.0
    x[2, 4] = -x[2, 3]
    x[5, 256:] = 0.0
    for cols in (6, 4, 2):
        run_case(be, O.Q4_K, n, rows, cols, x=x[:cols].copy())
        run_case(be, O.Q6_K, n, rows, cols, x=x[:cols].copy())


def test_empty(be):
    n, rows = 256, 8
    w, _ = make(O.Q4_K, n, rows, 1)
    wd = torch.from_numpy(w).cuda()
    x = torch.zeros((0, n), dtype=torch.float32, device="cuda")
    out = be.mul_mat(wd, O.Q4_K, n, x)
    assert out.shape == (0, rows)


@pytest.mark.parametrize("name,ty,n,rows", [
    ("q/o", O.Q4_K, 4096, 4096),
    ("k/v", O.Q4_K, 4096, 1024),
    ("gate/up", O.Q4_K, 4096, 14336),
    ("down", O.Q6_K, 14336, 4096),
    ("cfg1", O.Q4_0, 4096, 4096),
    ("q4_0 wide (separate Q8_0 quantization)", O.Q4_0, 4096, 14336),
])
@pytest.mark.parametrize("cols", [1, 2, 3, 4, 5, 8])
def test_llama3_decode_shapes(be, name, ty, n, rows, cols):
    if ty == O.Q4_0 and cols > 1:
        pytest.skip("the Q4_0 configurations are batch 1")
    run_case(be, ty, n, rows, cols, seed=0, check_sub=(cols <= 2))


@pytest.mark.parametrize("cols", [3, 5, 6, 7])
def test_padding_columns_not_stored(be, cols):
    """Batches that are not a kernel width (3 -> 4, 5..7 -> 8 columns): the
    padding columns must not be written.  dst is the first `cols` rows of an
    8-row buffer; the rows after it keep their canary values.  K = 4096 (one
    wavefront per row) and 14336 output rows, the decode shapes."""
    import ghip
    k, n = 4096, 14336
    g = torch.Generator(device="cuda").manual_seed(cols)
    w = be.quantize(torch.randn((n, k), device="cuda", generator=g) * 0.02, ghip.Q4_K)
    x = torch.randn((cols, k), device="cuda", generator=g)
    full = torch.full((8, n), 12345.0, device="cuda")
    be.mul_mat(w, ghip.Q4_K, k, x, out=full[:cols])
    torch.cuda.synchronize()
    assert bool((full[cols:] == 12345.0).all())
    assert torch.isfinite(full[:cols]).all()


def test_unsupported_type_raises(be):
    import ghip
    # TQ1_0 (type 34, 54-byte super-blocks) is the reference's documented
    # refusal (compute.rs:1456-1464): a status, no fallback
    ghip.BLOCK.setdefault(34, (256, 54))
    w = torch.zeros((8, 54), dtype=torch.uint8, device="cuda")
    x = torch.zeros((1, 256), dtype=torch.float32, device="cuda")
    with pytest.raises(ghip.GhipError, match="not supported"):
        be.mul_mat(w, 34, 256, x)


# ---------------------------------------------------------------- prefill GEMM
@pytest.mark.parametrize("n,rows,cols", [(256, 32, 16), (512, 136, 37), (1024, 128, 128),
                                         (768, 200, 130), (4096, 256, 64)])
def test_gemm_q4K_small(be, n, rows, cols):
    """Q4_K with >= 16 activation rows takes the int8-MFMA GEMM; tile edges in
    both M (tokens) and N (weight rows)."""
    run_case(be, O.Q4_K, n, rows, cols, seed=rows)


@pytest.mark.parametrize("n,rows,cols", [(256, 32, 16), (512, 136, 37), (1024, 128, 128), (768, 200, 130),
                                         (4096, 300, 64), (2048, 64, 16)])
def test_gemm_q5K_small(be, n, rows, cols):
    """Q5_K with >= 16 activation rows takes the wide int8-MFMA GEMM with the
    fifth-bit plane (split K when the tiles are few); tile edges in tokens and
    rows; Q8_K bytes and int32 {iacc, imin} sub-sums bit-exact."""
    run_case(be, O.Q5_K, n, rows, cols, seed=rows + 7)


def test_gemm_q5K_extreme_blocks(be):
    """Q5_K blocks at the ends of every field (6-bit scales and mins 63, all
    codes 31 with qh all ones, or 0) against the oracle: the fifth-bit plane
    2 * sc * bit stays within int8 and the sums exact."""
    rng = np.random.default_rng(11)
    n, rows, cols = 1024, 64, 32
    w = rng.integers(0, 256, size=(rows, O.row_size(O.Q5_K, n)), dtype=np.uint8)
    blk = w.reshape(rows, n // 256, 176)
    blk[:, :, 0:2] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)  # finite d, dmin
    blk[:, :, 2:4] = np.frombuffer(np.float16(0.02).tobytes(), np.uint8)
    blk[::2, :, 4:16] = 0xFF                      # every scale and min 63
    blk[::4, :, 16:176] = 0xFF                    # codes 31
    blk[1::4, :, 16:176] = 0                      # codes 0
    x = np.random.default_rng(12).standard_normal((cols, n)).astype(np.float32)
    run_case(be, O.Q5_K, n, rows, cols, x=x, w=w)


@pytest.mark.parametrize("n,rows,cols", [(512, 136, 64), (1024, 200, 100), (768, 128, 130), (4096, 256, 64),
                                         (512, 8, 200)])
def test_gemm_q6K_small(be, n, rows, cols):
    """Q6_K with >= 64 activation rows takes the f16-MFMA GEMM (repacked
    weights, exact split-scale planes); tile edges in tokens and rows; int32
    sub-sums bit-exact."""
    run_case(be, O.Q6_K, n, rows, cols, seed=rows + cols)


def test_gemm_q6K_prefill_down(be):
    """The Q4_K_M down projection at 512 tokens: 14336 -> 4096 Q6_K.  The GPU
    computes the whole product; the oracle checks a 512-row slice, plus the
    sub-sums of 32 of those rows."""
    tokens, n, rows = 512, 14336, 4096
    w, x = make(O.Q6_K, n, rows, tokens, seed=5)
    sl = slice(1000, 1512)
    wsl = w[sl]
    print(f"gemm q6_K tokens={tokens} n={n} rows={rows}", flush=True)
    got = be.mul_mat(torch.from_numpy(w).cuda(), O.Q6_K, n, torch.from_numpy(x).cuda()).cpu().numpy()
    want, _, _ = O.mul_mat(O.Q6_K, wsl, n, 512, x, tokens)
    err = rel_err(got[:, sl], want)
    assert err <= TOL, f"rel_err {err:.3e}"
    w32 = np.ascontiguousarray(wsl[:32])
    sub = be.mul_mat_subsums(torch.from_numpy(w32).cuda(), O.Q6_K, n, torch.from_numpy(x).cuda()).cpu().numpy()
    _, _, want_sub = O.mul_mat(O.Q6_K, w32, n, 32, x, tokens, want_subsums=True)
    assert np.array_equal(sub, want_sub)


@pytest.mark.parametrize("tokens,n,rows", [(128, 4096, 4096), (512, 4096, 14336), (2048, 4096, 4096)])
def test_gemm_q4K_prefill_shapes(be, tokens, n, rows):
    """Config 3 shapes.  The GPU computes the whole product; the oracle checks
    a 512-row slice of the weights (every token, every super-block), plus the
    sub-sums of 64 of those rows."""
    w, x = make(O.Q4_K, n, rows, tokens, seed=3)
    sl = slice(rows // 3, rows // 3 + 512) if rows > 512 else slice(0, rows)
    wsl = w[sl]
    nr = wsl.shape[0]
    print(f"gemm tokens={tokens} n={n} rows={rows}", flush=True)
    got = be.mul_mat(torch.from_numpy(w).cuda(), O.Q4_K, n, torch.from_numpy(x).cuda()).cpu().numpy()
    want, route, _ = O.mul_mat(O.Q4_K, wsl, n, nr, x, tokens)
    assert route == O.ROUTE_REPACK
    err = rel_err(got[:, sl], want)
    assert err <= TOL, f"rel_err {err:.3e}"
    w64 = np.ascontiguousarray(wsl[:64])
    sub = be.mul_mat_subsums(torch.from_numpy(w64).cuda(), O.Q4_K, n, torch.from_numpy(x).cuda()).cpu().numpy()
    _, _, want_sub = O.mul_mat(O.Q4_K, w64, n, 64, x, tokens, want_subsums=True)
    assert np.array_equal(sub, want_sub)


@pytest.mark.parametrize("n,rows,cols", [(1024, 204, 16), (2048, 204, 130), (512, 12, 64), (4096, 4100, 64)])
def test_gemm_q4K_rows_not_multiple_of_8(be, n, rows, cols):
    """Q4_K with N % 8 != 0 and >= 16 activation rows: the reference takes the
    tiled route (compute.rs:1596) with quantize_row_q8_K_ref activations for
    every row (no 4x8 values); the GPU runs its GEMM on those bytes.  The
    activation bytes are compared in full; at 4100 rows the oracle checks the
    last 516 rows (the ragged tile edge) and the sub-sums of the last 4."""
    w, x = make(O.Q4_K, n, rows, cols, seed=rows + cols)
    sl = slice(max(0, rows - 516), rows)
    wsl = np.ascontiguousarray(w[sl])
    nr = wsl.shape[0]
    print(f"gemm q4_K n={n} rows={rows} cols={cols}", flush=True)
    wd, xd = torch.from_numpy(w).cuda(), torch.from_numpy(x).cuda()
    got = be.mul_mat(wd, O.Q4_K, n, xd).cpu().numpy()
    want, route, _ = O.mul_mat(O.Q4_K, wsl, n, nr, x, cols)
    assert route == (O.ROUTE_TILED if nr % 8 else O.ROUTE_REPACK)
    act = be.mul_mat_act(wd, O.Q4_K, n, xd).cpu().numpy().reshape(-1)
    assert np.array_equal(act, O.mul_mat_act(O.Q4_K, n, rows, x, cols))
    assert np.array_equal(act, np.concatenate([O.quantize(O.Q8_K, x[c], kind="quantize_row_q8_K_ref")
                                               for c in range(cols)]))
    err = rel_err(got[:, sl], want)
    assert err <= TOL, f"rel_err {err:.3e}"
    w4 = np.ascontiguousarray(w[rows - 4:])
    sub = be.mul_mat_subsums(torch.from_numpy(w4).cuda(), O.Q4_K, n, xd).cpu().numpy()
    _, _, want_sub = O.mul_mat(O.Q4_K, w4, n, 4, x, cols, want_subsums=True)
    assert np.array_equal(sub, want_sub)


@pytest.mark.parametrize("ty", [O.Q4_0, O.Q5_0, O.Q8_0])
@pytest.mark.parametrize("n,rows,cols", [(256, 64, 32), (1024, 200, 100), (2880, 136, 130), (4096, 256, 64)])
def test_gemm_q8_family(be, ty, n, rows, cols):
    """Q4_0 / Q5_0 / Q8_0 with >= 32 f32 activation rows take the int8-MFMA
    GEMM (one exact 32-block dot per MFMA); K not a multiple of 128 (2880)
    pads with zeros; int32 block dots bit-exact."""
    run_case(be, ty, n, rows, cols, seed=rows + cols + ty)


def test_gemm_q8_family_registered(be):
    """A registered Q4_0 weight (its int8 codes kept on the device) gives the
    same bits as the per-call repack."""
    n, rows, cols = 4096, 512, 96
    w, x = make(O.Q4_0, n, rows, cols, seed=9)
    wd, xd = torch.from_numpy(w).cuda(), torch.from_numpy(x).cuda()
    print(f"gemm q8 registered n={n} rows={rows} cols={cols}", flush=True)
    before = be.mul_mat(wd, O.Q4_0, n, xd).clone()
    be.register_weight(wd, O.Q4_0, n)
    assert torch.equal(be.mul_mat(wd, O.Q4_0, n, xd), before)
    be.unregister_weight(wd, O.Q4_0, n)


@pytest.mark.parametrize("ty,n,rows,cols", [
    (O.Q4_K, 1280, 100, 4),    # 5 super-blocks: slices of 4 + 1, a partial 64-row tile
    (O.Q4_K, 1536, 1000, 7),   # 6 super-blocks: the last slice one 2-block step
    (O.Q4_K, 256, 64, 8),      # one slice: no partials
    (O.Q4_K, 7168, 300, 5),    # 28 super-blocks: slices of 8
    (O.Q6_K, 1792, 70, 4),     # 7 super-blocks
    (O.Q6_K, 8192, 130, 7),    # 32 super-blocks: slices of 8
    (O.Q6_K, 256, 16, 8),
    (O.Q4_K, 16384, 40, 5),    # 64 super-blocks: past the whole-K LDS images, split K on every route
    (O.Q6_K, 16384, 24, 6),
])
@pytest.mark.parametrize("route", ["whole_k", "split_k"])
def test_split_k_decode(be, monkeypatch, route, ty, n, rows, cols):
    """The 4..8-row decode kernels for Q4_K and Q6_K.  whole_k (the default,
    ghip_sq_*): one wavefront per 2-super-block K-slice of a workgroup that
    owns whole rows, the ready Q8_K rows copied into each wavefront's LDS
    image, the slices' partials added in wavefront order; 1..16 wavefronts,
    a ragged last slice and 16-row tiles.  split_k (GHIP_SQ=0; Q4_K forced
    onto it below 8192 weight rows): the activation slice quantized inside
    each workgroup, the K-slices' partials added in order by ghip_sk_reduce;
    ragged slices, steps and row tiles.  Q8_K bytes and int32 sub-sums
    bit-exact."""
    if route == "split_k":
        monkeypatch.setenv("GHIP_SQ", "0")
        monkeypatch.setenv("GHIP_SK_MIN_ROWS", "1")
    print(f"{route} decode type={ty} n={n} rows={rows} cols={cols}", flush=True)
    run_case(be, ty, n, rows, cols, seed=rows + cols)


@pytest.mark.parametrize("ty,n,rows,cols", [
    (O.Q4_K, 14336, 90, 8),   # 56 super-blocks: 4-block slices, 14 wavefronts
    (O.Q6_K, 14336, 40, 6),
    (O.Q4_K, 8448, 33, 4),    # 33 super-blocks: 4-block slices, the last one 1 block
    (O.Q4_K, 13312, 20, 5),   # 52 super-blocks: 13 wavefronts
])
def test_whole_k_decode_long_rows(be, ty, n, rows, cols):
    """The whole-K decode kernels on rows of 33..56 super-blocks (4-block
    slices per wavefront, up to 14 wavefronts and 159 KB of LDS) against the
    oracle; Q8_K bytes and sub-sums bit-exact."""
    print(f"whole-K long rows type={ty} n={n} rows={rows} cols={cols}", flush=True)
    run_case(be, ty, n, rows, cols, seed=rows + cols + 1)


@pytest.mark.parametrize("ty,n", [(O.Q4_K, 4096), (O.Q6_K, 4096)])
def test_whole_k_tiles_per_workgroup(be, monkeypatch, ty, n):
    """One or two 16-row tiles per workgroup (GHIP_SQ_T) give the same bits:
    the tile count changes which workgroup computes a row, not its sums."""
    w, x = make(ty, n, 2000, 8, seed=4)
    wd, xd = torch.from_numpy(w).cuda(), torch.from_numpy(x).cuda()
    print(f"whole-K tiles per workgroup type={ty}", flush=True)
    monkeypatch.setenv("GHIP_SQ_T", "1")
    want = be.mul_mat(wd, ty, n, xd).clone()
    monkeypatch.setenv("GHIP_SQ_T", "2")
    assert torch.equal(be.mul_mat(wd, ty, n, xd), want)


def test_split_k_tiles_per_workgroup(be, monkeypatch):
    """Few workgroups (GHIP_SK_WGS): each walks several tiles with the next
    step's weights in flight; same bits as one tile per workgroup."""
    monkeypatch.setenv("GHIP_SQ", "0")
    w, x = make(O.Q4_K, 4096, 14336, 8, seed=3)
    wd, xd = torch.from_numpy(w).cuda(), torch.from_numpy(x).cuda()
    print("split-K tiles per workgroup", flush=True)
    want = be.mul_mat(wd, O.Q4_K, 4096, xd).clone()
    for wgs in ("8", "100", "100000"):
        monkeypatch.setenv("GHIP_SK_WGS", wgs)
        assert torch.equal(be.mul_mat(wd, O.Q4_K, 4096, xd), want)


@pytest.mark.parametrize("ty,n,rows", [(O.Q4_K, 4096, 14336), (O.Q6_K, 14336, 4096)])
def test_split_k_repeat_and_graph(be, ty, n, rows):
    """The per-tile counters return to zero after every call: repeated calls,
    and replays of a captured graph between eager calls, give the same bits."""
    w, x = make(ty, n, rows, 8, seed=5)
    wd, xd = torch.from_numpy(w).cuda(), torch.from_numpy(x).cuda()
    print(f"split-K repeat type={ty} n={n} rows={rows}", flush=True)
    first = be.mul_mat(wd, ty, n, xd).clone()
    for _ in range(3):
        assert torch.equal(be.mul_mat(wd, ty, n, xd), first)
    out = torch.empty_like(first)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        be.mul_mat(wd, ty, n, xd, out=out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        be.mul_mat(wd, ty, n, xd, out=out)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first)
        assert torch.equal(be.mul_mat(wd, ty, n, xd), first)
    want, _, _ = O.mul_mat(ty, w, n, rows, x, 8)
    assert rel_err(first.cpu().numpy(), want) <= TOL


@pytest.mark.parametrize("rows,wgs", [(14336, "256"), (8200, "256"), (9000, "7"), (8192, "100000")])
def test_gemv_persistent_grid(be, monkeypatch, rows, wgs):
    """Q4_K at one activation row from 8192 weight rows on the persistent grid
    (GHIP_GEMV_PERSIST=1; GHIP_GEMV_WGS workgroups, every team an equal run of
    rows; teams past the last row compute nothing): ragged row counts and grid
    sizes against the oracle, sub-sums through the non-persistent kernel."""
    monkeypatch.setenv("GHIP_GEMV_PERSIST", "1")
    monkeypatch.setenv("GHIP_GEMV_WGS", wgs)
    run_case(be, O.Q4_K, 4096, rows, 1, seed=rows)


@pytest.mark.parametrize("ty,ne02,ne03,ne12,ne13,m,perm", [
    (O.Q4_K, 1, 1, 3, 1, 5, False),    # one weight plane broadcast to 3 activation planes (r2 = 3)
    (O.Q4_K, 2, 1, 4, 2, 4, False),    # r2 = 2, r3 = 2
    (O.Q8_0, 2, 2, 2, 2, 3, True),     # one-to-one planes, src1 planes not contiguous
    (O.Q6_K, 1, 2, 2, 4, 1, True),
    (O.Q4_0, 3, 1, 3, 1, 40, False),   # 40 rows: the prefill GEMM per plane
])
def test_batched_broadcast(be, ty, ne02, ne03, ne12, ne13, m, perm):
    """Batched MUL_MAT (forward_mul_mat, compute.rs:1440-1450): dst plane
    (i12, i13) = src0 plane (i12 / r2, i13 / r3) x src1 plane (i12, i13).
    Every plane against the oracle's 2-D MUL_MAT of the planes it reads, to
    the matmul bar."""
    import ctypes as C
    import ghip
    k, n = 512, 96
    rng = np.random.default_rng(ne12 * 10 + ne13)
    wf = (rng.standard_normal((ne03, ne02, n, k)) * 0.02).astype(np.float32)
    wq = np.stack([np.stack([O.quantize(ty, wf[i3, i2]).reshape(n, -1) for i2 in range(ne02)]) for i3 in range(ne03)])
    x = rng.standard_normal((ne13, ne12, m, k)).astype(np.float32)
    wd = torch.from_numpy(wq).cuda()
    if perm:  # planes laid out [ne12][ne13] in memory, viewed as [ne13][ne12]
        xd = torch.from_numpy(np.ascontiguousarray(x.transpose(1, 0, 2, 3))).cuda().permute(1, 0, 2, 3)
    else:
        xd = torch.from_numpy(x).cuda()
    out = torch.full((ne13, ne12, m, n), float("nan"), device="cuda")
    a, b, d = ghip.describe(wd, ty, k), ghip.describe(xd, ghip.F32), ghip.describe(out, ghip.F32)
    assert list(d.ne) == [n, m, ne12, ne13] and list(b.ne) == [k, m, ne12, ne13]
    assert ghip.lib().ghip_supports_op(ghip.OP_MUL_MAT, C.byref(d), (C.POINTER(ghip.Tensor) * 2)(C.pointer(a), C.pointer(b)), 2) == 1
    be._check(ghip.lib().ghip_mul_mat(be._ctx, C.byref(a), C.byref(b), C.byref(d), ghip._stream()), "ghip_mul_mat")
    got = out.cpu().numpy()
    r2, r3 = ne12 // ne02, ne13 // ne03
    for i3 in range(ne13):
        for i2 in range(ne12):
            want, _, _ = O.mul_mat(ty, wq[i3 // r3, i2 // r2], k, n, x[i3, i2], m)
            assert rel_err(got[i3, i2], want.reshape(m, n)) <= TOL, (i3, i2)


def test_batched_shape_errors(be):
    """ne12 not a multiple of ne02, and a dst whose planes differ from src1's"""
    import ctypes as C
    import ghip
    k, n, m = 256, 32, 2
    wd = torch.zeros((2, n, ghip.row_size(ghip.Q8_0, k)), dtype=torch.uint8, device="cuda")
    for ne12, dplanes, msg in ((3, 3, "multiples of src0"), (2, 1, "dst must be F32")):
        xd = torch.zeros((ne12, m, k), device="cuda")
        out = torch.zeros((dplanes, m, n), device="cuda")
        a, b, d = ghip.describe(wd, ghip.Q8_0, k), ghip.describe(xd, ghip.F32), ghip.describe(out, ghip.F32)
        with pytest.raises(ghip.GhipError, match=msg):
            be._check(ghip.lib().ghip_mul_mat(be._ctx, C.byref(a), C.byref(b), C.byref(d), ghip._stream()), "ghip_mul_mat")


@pytest.mark.parametrize("cols", [9, 11, 15])
def test_q4K_long_k_9_to_15_rows(be, cols):
    """Q4_K down projection (K = 14336) at 9-15 activation rows: the
    matrix-core decode kernel's 16-column LDS image does not fit there, so
    the rows go to the whole-row kernels in groups of 8 columns.  The oracle
    takes the reference's tiled route from 8 columns; the bar is 1e-5 or the
    gap between the reference's own two routes on these inputs (row vec_dot
    per column against the tiled kernel), whichever is larger."""
    n, rows = 14336, 512
    w, x = make(O.Q4_K, n, rows, cols, cols)
    want, route, want_sub = O.mul_mat(O.Q4_K, w, n, rows, x, cols, want_subsums=True)
    vd = np.concatenate([O.mul_mat(O.Q4_K, w, n, rows, x[c:c + 1], 1)[0] for c in range(cols)])
    gap = rel_err(vd.reshape(cols, rows), want.reshape(cols, rows))
    wd, xd = torch.from_numpy(w).cuda(), torch.from_numpy(x).cuda()
    print(f"case q4_K n={n} rows={rows} cols={cols} route={route} route gap {gap:.2e}", flush=True)
    got = be.mul_mat(wd, O.Q4_K, n, xd).cpu().numpy()
    assert np.array_equal(be.mul_mat_subsums(wd, O.Q4_K, n, xd).cpu().numpy(), want_sub)
    err = rel_err(got, want.reshape(got.shape))
    assert err <= max(TOL, gap), (err, gap)
