"""GPU parity of GGML_OP_FLASH_ATTN_EXT (f16 K/V) against the CPU oracle.

Bar: within 2e-3 max-abs of the reference path.  The
oracle follows the reference's dispatch (split-KV for single-row decode with
S >= 512, tiled for >= 64 query rows, one_chunk otherwise), pinned bit-exact
on parity/fa_ref.bin and fa_probe.bin (test_oracle_golden.py).
"""
import numpy as np
import pytest

import oracle_lib as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 2e-3


@pytest.fixture(scope="module")
def be():
    import ghip
    b = ghip.Backend(0)
    yield b
    b.close()


def causal_mask(T, S):
    m = np.zeros((T, S), dtype=np.float16)
    for t in range(T):
        m[t, S - T + t + 1:] = -np.inf
    return m


def run(be, H, Hkv, D, T, S, mask="causal", sinks=False, softcap=0.0, max_bias=0.0, seed=0, n_chunks=8):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((H, T, D)).astype(np.float32)
    k = rng.standard_normal((Hkv, S, D)).astype(np.float16)
    v = rng.standard_normal((Hkv, S, D)).astype(np.float16)
    m = causal_mask(T, S) if mask == "causal" else (np.zeros((T, S), np.float16) if mask == "zero" else None)
    sk = rng.standard_normal(H).astype(np.float32) if sinks else None
    scale = 1.0 / np.sqrt(D)
    want, path = O.flash_attn_ext(q, k, v, m, sk, scale, max_bias, softcap, n_chunks=n_chunks)
    print(f"fa H={H} Hkv={Hkv} D={D} T={T} S={S} mask={mask} path={path}", flush=True)
    t = lambda a: torch.from_numpy(a).cuda() if a is not None else None
    got = be.flash_attn_ext(t(q), t(k), t(v), t(m), t(sk), scale, max_bias, softcap).cpu().numpy()
    err = float(np.max(np.abs(got - want)))
    assert err <= TOL, f"max-abs {err:.3e}"
    return err


@pytest.mark.parametrize("T,S", [(1, 64), (1, 100), (1, 600), (3, 40), (5, 700), (32, 96), (64, 64), (70, 130)])
def test_small(be, T, S):
    run(be, 4, 2, 64, T, S)
    run(be, 8, 2, 128, T, S, seed=1)


def test_variants(be):
    run(be, 4, 4, 128, 2, 300, mask=None)
    run(be, 4, 1, 64, 65, 200, sinks=True)
    run(be, 4, 2, 64, 70, 200, softcap=15.0)
    run(be, 8, 2, 64, 64, 128, max_bias=8.0, mask="zero")
    run(be, 4, 2, 128, 1, 513, sinks=True)


@pytest.mark.parametrize("H,Hkv,D,T,S", [(4, 4, 128, 100, 301), (6, 2, 128, 100, 258), (6, 2, 64, 130, 67),
                                         (8, 1, 128, 64, 150), (7, 1, 64, 96, 333), (16, 2, 128, 200, 1031)])
def test_head_groups(be, H, Hkv, D, T, S):
    """Tiled route for every head-group size: workgroups of G heads times
    ceil(4 / G) query tiles, ragged key counts and ragged query tiles."""
    run(be, H, Hkv, D, T, S, seed=H + T)


def test_fully_masked_rows(be):
    """Rows whose keys are all masked produce zeros (S == 0 -> S_inv = 0)."""
    H, Hkv, D, T, S = 4, 2, 64, 4, 80
    rng = np.random.default_rng(9)
    q = rng.standard_normal((H, T, D)).astype(np.float32)
    k = rng.standard_normal((Hkv, S, D)).astype(np.float16)
    v = rng.standard_normal((Hkv, S, D)).astype(np.float16)
    m = np.zeros((T, S), dtype=np.float16)
    m[1, :] = -np.inf
    want, _ = O.flash_attn_ext(q, k, v, m, None, 0.125)
    got = be.flash_attn_ext(*(torch.from_numpy(a).cuda() for a in (q, k, v, m)), None, 0.125).cpu().numpy()
    assert np.all(got[1] == 0.0)
    assert np.max(np.abs(got - want)) <= TOL


@pytest.mark.parametrize("T", [1, 512])
def test_config5(be, T):
    """Config 5: 32 query / 8 KV heads, D = 128, KV 8192, causal chunk at the
    end of the cache (decode T = 1, prefill T = 512)."""
    run(be, 32, 8, 128, T, 8192, seed=5, n_chunks=16)


def run_general(be, H, Hkv, DK, DV, T, S, kv=np.float16, sinks=False, seed=0, n_chunks=8):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((H, T, DK)).astype(np.float32)
    k = rng.standard_normal((Hkv, S, DK)).astype(kv)
    v = rng.standard_normal((Hkv, S, DV)).astype(kv)
    m = causal_mask(T, S)
    sk = rng.standard_normal(H).astype(np.float32) if sinks else None
    scale = 1.0 / np.sqrt(DK)
    want, path = O.flash_attn_ext(q, k, v, m, sk, scale, 0.0, 0.0, n_chunks=n_chunks)
    print(f"fa general H={H} Hkv={Hkv} DK={DK} DV={DV} T={T} S={S} kv={np.dtype(kv).name} path={path}", flush=True)
    t = lambda a: torch.from_numpy(a).cuda() if a is not None else None
    got = be.flash_attn_ext(t(q), t(k), t(v), t(m), t(sk), scale).cpu().numpy()
    err = float(np.max(np.abs(got - want)))
    assert err <= TOL, f"max-abs {err:.3e}"


@pytest.mark.parametrize("H,Hkv,DK,DV,T,S,kv", [
    (8, 2, 256, 256, 5, 300, np.float16),    # D = 256, row walk (f16 accumulator)
    (8, 2, 256, 256, 70, 200, np.float16),   # D = 256, tiled route
    (4, 2, 64, 128, 3, 90, np.float16),      # DK != DV
    (4, 2, 192, 128, 66, 130, np.float16),   # DK != DV, tiled route
    (4, 2, 32, 32, 40, 100, np.float16),
    (4, 2, 64, 64, 10, 80, np.float32),      # F32 K/V, row walk
    (4, 1, 128, 128, 64, 128, np.float32),   # F32 K/V, tiled route
    (32, 2, 64, 64, 4, 120, np.float16),     # H / H_kv = 16
    (16, 1, 80, 80, 1, 700, np.float16),     # split-KV route shape, head size 80
])
def test_general_shapes(be, H, Hkv, DK, DV, T, S, kv):
    """Shapes outside the tuned kernels (F32 K/V, DK != DV, head sizes other
    than 64 / 128, H / H_kv > 8) take the general row walk, still within 2e-3
    of the oracle's route for the shape."""
    run_general(be, H, Hkv, DK, DV, T, S, kv, sinks=(T % 2 == 1))


@pytest.mark.parametrize("T,S,m2,m3", [
    (1, 600, 2, 1),    # split-KV shape, per-head mask planes (row walk, fp32)
    (1, 600, 1, 2),    # split-KV decode kernel, per-sequence planes
    (5, 300, 8, 2),    # one-chunk walk (f16 accumulator)
    (70, 200, 4, 1),   # tiled route on the matrix cores, per-head planes
    (70, 200, 1, 1),
])
def test_mask_planes_and_sequences(be, T, S, m2, m3):
    """The rest of the operand contract (flash_attn.rs:30-37, :298): two
    sequences (ne3 = 2) with their own q, k and v planes, and mask planes
    broadcast to heads by h % ne2 and to sequences by i3 % ne3.  Each
    (sequence, head) is checked against the oracle's route for its shape on
    exactly the mask plane it must read."""
    H, Hkv, D, n_seq = 8, 2, 128, 2
    G = H // Hkv
    rng = np.random.default_rng(T * 1000 + m2 * 10 + m3)
    q = rng.standard_normal((n_seq, H, T, D)).astype(np.float32)
    k = rng.standard_normal((n_seq, Hkv, S, D)).astype(np.float16)
    v = rng.standard_normal((n_seq, Hkv, S, D)).astype(np.float16)
    m = np.zeros((m3, m2, T, S), dtype=np.float16)
    for i3 in range(m3):
        for i2 in range(m2):  # a different causal window per plane
            off = int(rng.integers(0, S // 3))
            for t in range(T):
                m[i3, i2, t, S - T + t + 1 - off:] = -np.inf
            m[i3, i2] += (rng.standard_normal((T, S)) * 0.5).astype(np.float16)
    sk = rng.standard_normal(H).astype(np.float32)
    scale = 1.0 / np.sqrt(D)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    got = be.flash_attn_ext(t(q), t(k), t(v), t(m), t(sk), scale).cpu().numpy()
    assert got.shape == (n_seq, T, H, D)
    worst = 0.0
    for i3 in range(n_seq):
        for h in range(H):
            want, path = O.flash_attn_ext(q[i3, h:h + 1], k[i3, h // G:h // G + 1], v[i3, h // G:h // G + 1],
                                          m[i3 % m3, h % m2], sk[h:h + 1], scale, 0.0, 0.0, n_chunks=8)
            worst = max(worst, float(np.max(np.abs(got[i3, :, h:h + 1] - want))))
    print(f"fa planes T={T} S={S} m2={m2} m3={m3} path={path} max-abs {worst:.2e}", flush=True)
    assert worst <= TOL


@pytest.mark.parametrize("T,S,m2", [(96, 640, 1), (70, 333, 2), (512, 2048, 1)])
def test_mask_tile_classes(be, T, S, m2):
    """The tiled route classifies each (32-query, 64-key) mask tile: all +-0
    (no mask loads), all -inf (no work), or mixed.  A mask made of such tiles
    (whole query blocks masked to -inf, -0.0 tiles, ragged T and S) gives the
    oracle's result, and the same bits as with the classes switched off
    (GHIP_FA_MASK_SCAN=0)."""
    import os
    H, Hkv, D = 8, 2, 128
    rng = np.random.default_rng(T + S + m2)
    q = rng.standard_normal((H, T, D)).astype(np.float32)
    k = rng.standard_normal((Hkv, S, D)).astype(np.float16)
    v = rng.standard_normal((Hkv, S, D)).astype(np.float16)
    m = np.zeros((m2, T, S), dtype=np.float16)
    for p2 in range(m2):
        for qb in range((T + 31) // 32):
            for tl in range((S + 63) // 64):
                c = int(rng.integers(0, 4))
                blk = m[p2, 32 * qb:32 * qb + 32, 64 * tl:64 * tl + 64]
                if c == 1:
                    blk[:] = -np.inf
                elif c == 2:
                    blk[:] = np.float16(-0.0)
                elif c == 3:
                    blk[:] = (rng.standard_normal(blk.shape) * 0.5).astype(np.float16)
        m[p2, 32:64, :] = -np.inf  # a whole query block with no visible key
    mm = m if m2 > 1 else m[0]
    scale = 1.0 / np.sqrt(D)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    outs = []
    for flag in ("0", "1"):
        os.environ["GHIP_FA_MASK_SCAN"] = flag
        try:
            outs.append(be.flash_attn_ext(t(q), t(k), t(v), t(mm), None, scale).cpu().numpy())
        finally:
            del os.environ["GHIP_FA_MASK_SCAN"]
    assert np.array_equal(outs[0], outs[1])
    assert np.all(outs[1][32:64] == 0.0)
    for h in range(H):
        want, _ = O.flash_attn_ext(q[h:h + 1], k[h // (H // Hkv):h // (H // Hkv) + 1],
                                   v[h // (H // Hkv):h // (H // Hkv) + 1], m[h % m2], None, scale, n_chunks=8)
        err = float(np.max(np.abs(outs[1][:, h:h + 1] - want)))
        assert err <= TOL, f"head {h}: max-abs {err:.3e}"


@pytest.mark.parametrize("sinks", [False, True])
def test_merge_preload_four(be, sinks):
    """At most 4 KV slices (T = 512, 32 / 8 heads: 4 slices) the merge loads
    exactly the slices it sums (ghip_fa_merge_rows_p4): the same bits as the
    16-slice preload (GHIP_FA_MERGE_P4=0), and the oracle's result."""
    import os
    H, Hkv, D, T, S = 32, 8, 128, 512, 2048
    rng = np.random.default_rng(5 + sinks)
    q = rng.standard_normal((H, T, D)).astype(np.float32)
    k = rng.standard_normal((Hkv, S, D)).astype(np.float16)
    v = rng.standard_normal((Hkv, S, D)).astype(np.float16)
    m = np.zeros((T, S), dtype=np.float16)
    for i in range(T):
        m[i, S - T + i + 1:] = -np.inf
    sk = (rng.standard_normal(H) * 2.0).astype(np.float32) if sinks else None
    scale = 1.0 / np.sqrt(D)
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()
    print(f"fa merge preload 4 sinks={sinks}", flush=True)
    outs = []
    for flag in ("0", "1"):
        os.environ["GHIP_FA_MERGE_P4"] = flag
        try:
            outs.append(be.flash_attn_ext(t(q), t(k), t(v), t(m), t(sk), scale).cpu().numpy())
        finally:
            del os.environ["GHIP_FA_MERGE_P4"]
    assert np.array_equal(outs[0], outs[1])
    for h in (0, 13, 31):
        g = h // (H // Hkv)
        want, _ = O.flash_attn_ext(q[h:h + 1], k[g:g + 1], v[g:g + 1], m, None if sk is None else sk[h:h + 1], scale,
                                   n_chunks=8)
        err = float(np.max(np.abs(outs[1][:, h:h + 1] - want)))
        assert err <= TOL, f"head {h}: max-abs {err:.3e}"


@pytest.mark.parametrize("T,S,D,masked,sinks", [(96, 640, 128, True, True), (130, 1000, 64, False, False),
                                                (64, 300, 128, True, False), (200, 2048, 64, True, True)])
def test_single_slice_direct(be, monkeypatch, T, S, D, masked, sinks):
    """One KV slice (GHIP_FA_WGS=1 forces it at these sizes; long prefills
    get it by themselves): the forward kernel writes the normalized rows,
    no partials and no merge launch.  Same bits as the partial-and-merge
    route (GHIP_FA_DIRECT=0), and the oracle's result."""
    H, Hkv = 8, 2
    rng = np.random.default_rng(T + S + D + 1)
    q = rng.standard_normal((H, T, D)).astype(np.float32)
    k = rng.standard_normal((Hkv, S, D)).astype(np.float16)
    v = rng.standard_normal((Hkv, S, D)).astype(np.float16)
    m = None
    if masked:
        m = np.zeros((T, S), dtype=np.float16)
        for i in range(T):
            m[i, S - T + i + 1:] = -np.inf
        m[:32, :] = -np.inf  # a query block with no visible key
    sk = (rng.standard_normal(H) * 2.0).astype(np.float32) if sinks else None
    scale = 1.0 / np.sqrt(D)
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()
    print(f"fa single slice T={T} S={S} D={D} masked={masked} sinks={sinks}", flush=True)
    monkeypatch.setenv("GHIP_FA_WGS", "1")
    outs = []
    for flag in ("0", "1"):
        monkeypatch.setenv("GHIP_FA_DIRECT", flag)
        outs.append(be.flash_attn_ext(t(q), t(k), t(v), t(m), t(sk), scale).cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    for h in (0, 5):
        g = h // (H // Hkv)
        want, _ = O.flash_attn_ext(q[h:h + 1], k[g:g + 1], v[g:g + 1], m, None if sk is None else sk[h:h + 1], scale,
                                   n_chunks=8)
        err = float(np.max(np.abs(outs[1][:, h:h + 1] - want)))
        assert err <= TOL, f"head {h}: max-abs {err:.3e}"
