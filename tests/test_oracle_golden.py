"""Pin the CPU oracle against the reference's golden fixtures and closed forms.

Each test names the reference test it mirrors.  These run on the CPU only.
"""
import numpy as np
import pytest

import fixtures as fx
import oracle_lib as O


def test_fp16_matches_ieee_rne():
    """fp32->fp16 RNE (half 2.7.1) against numpy's IEEE conversion, and the
    exact fp16->fp32 widening over all 65536 patterns."""
    L = O.lib()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([L.oracle_fp16_to_fp32(int(v)) for v in h[::7]], dtype=np.float32)
    w = want[::7]
    nan = np.isnan(w)
    assert np.array_equal(got[~nan].view(np.uint32), w[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()
    rng = np.random.default_rng(3)
    x = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(1e-5),   # subnormal halves
        rng.standard_normal(4000).astype(np.float32) * np.float32(100.0),
        (np.arange(2048, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -24),  # exact ties
        np.array([65504.0, 65520.0, 65519.99, -0.0, 1e9, 2.0 ** -25, 2.0 ** -26], dtype=np.float32),
    ])
    got = np.array([L.oracle_fp32_to_fp16(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))


def test_nearest_int_is_rne():
    L = O.lib()
    rng = np.random.default_rng(4)
    x = np.concatenate([rng.uniform(-300, 300, 3000).astype(np.float32),
                        np.arange(-20, 20, dtype=np.float32) + np.float32(0.5)])
    got = np.array([L.oracle_nearest_int(float(v)) for v in x])
    assert np.array_equal(got, np.rint(x).astype(np.int64))


def test_e8m0_closed_form():
    """quants.rs e8m0_scale_boundaries: every byte maps to 2^(x-128)."""
    L = O.lib()
    for x in range(256):
        want = np.float32(2.0 ** (x - 128))
        assert np.float32(L.oracle_e8m0_to_fp32_half(x)).view(np.uint32) == want.view(np.uint32)


QUANT_NAME = {O.Q4_0: "quantize_row_q4_0_ref", O.Q8_0: "quantize_row_q8_0_ref",
              O.Q4_K: "quantize_row_q4_K_ref", O.Q6_K: "quantize_row_q6_K_ref",
              O.Q8_K: "quantize_row_q8_K_ref", O.Q5_0: "quantize_row_q5_0_ref",
              O.Q5_K: "quantize_row_q5_K_ref", O.Q4_1: "quantize_row_q4_1_ref",
              O.Q5_1: "quantize_row_q5_1_ref", O.Q8_1: "quantize_row_q8_1"}


def test_quants_ref_bit_exact():
    """quants.rs:791 quants_bit_exact_vs_reference + quants_k.rs:2479
    k_quant_quantize_bit_exact_vs_reference, restricted to the hot-path types."""
    x = fx.ref_input(1024)
    secs = {tid: (q, deq) for (_, tid, n, q, deq) in fx.quant_sections("quants_ref.bin")}
    assert len(secs) == 12
    for tid, name in QUANT_NAME.items():
        q, deq = secs[tid]
        mine = O.quantize(tid, x, kind=name)
        assert np.array_equal(mine, q), f"type {tid}: quantized bytes differ"
        if tid != O.Q8_K and deq.any():
            got = O.dequantize(tid, q, 1024)
            assert np.array_equal(got.view(np.uint32), deq.view(np.uint32)), f"type {tid}: dequant differs"


def test_mxfp4_quantizer_and_dequant_bit_exact():
    """quants.rs fp4_dequant_bit_exact_vs_reference; the SECT sections also pin
    the upstream MXFP4 quantizer the reference lacks."""
    secs = [s for s in fx.quant_sections("quants_ref_fp4.bin") if s[1] == O.MXFP4]
    assert len(secs) == 4
    x = fx.ref_input(1024)
    for magic, tid, n, q, deq in secs:
        got = O.dequantize(O.MXFP4, q, n)
        assert np.array_equal(got.view(np.uint32), deq.view(np.uint32))
        if magic == 0x54434553:  # quantizer-produced section
            assert np.array_equal(O.quantize(O.MXFP4, x[:n]), q), f"mxfp4 quantizer n={n}"


@pytest.mark.parametrize("name", ["mulmat_ref_c1.bin", "mulmat_ref.bin"])
def test_mulmat_vec_dot_bit_exact(name):
    """vec_dot.rs:2378/2449 mulmat_(c1_)bit_exact_vs_reference for Q4_0/Q4_K/Q6_K.
    4 weight rows -> no repack; cols < 8 -> no tiled; so the row vec_dot route.
    Q4_0 with 3 columns takes llamafile tinyBLAS in the reference (out of scope):
    checked there within 1e-6 by the per-row vec_dot."""
    checked = 0
    for tid, n, rows, cols, xq, y, dst in fx.mulmat_sections(name):
        if tid not in (O.Q4_0, O.Q4_K, O.Q6_K):
            continue
        if tid == O.Q4_0 and cols >= 2:
            act = O.mul_mat_act(O.Q4_0, n, rows, y[:1], 1)
            out = np.zeros((cols, rows), dtype=np.float32)
            for c in range(cols):
                a = O.quantize(O.Q8_0, y[c], kind="quantize_row_q8_0")
                for r in range(rows):
                    w = xq[r * O.row_size(O.Q4_0, n):(r + 1) * O.row_size(O.Q4_0, n)]
                    out[c, r] = O.lib().oracle_vec_dot_q4_0_q8_0(n, O._p(w), O._p(a))
            err = np.max(np.abs(out - dst) / np.maximum(np.abs(dst), 1))
            assert err <= 1e-6
            del act
        else:
            out, route, _ = O.mul_mat(tid, xq, n, rows, y, cols)
            assert route == O.ROUTE_VECDOT
            assert np.array_equal(out.view(np.uint32), dst.view(np.uint32)), f"type {tid} {name}"
        checked += 1
    assert checked == 3


@pytest.mark.parametrize("name", ["mulmat_ref_c1.bin", "mulmat_ref.bin"])
def test_mulmat_q5_0_q8_0_q5_K_bit_exact(name):
    """The same dumps for Q5_0 (type 6), Q8_0 (type 8) and Q5_K (type 13): 4 rows,
    1 or 3 columns, so the row vec_dot (vec_dot.rs:661/732/928) -- for Q5_0/Q8_0
    with 3 columns the reference ran tinyBLAS_Q0, which keeps the vec_dot's
    lanes and fma order (tinyblas.rs:55-75): bit-exact either way."""
    seen = set()
    for tid, n, rows, cols, xq, y, dst in fx.mulmat_sections(name):
        if tid not in (O.Q5_0, O.Q8_0, O.Q5_K):
            continue
        out, route, sub = O.mul_mat(tid, xq, n, rows, y, cols, want_subsums=True)
        assert route == O.ROUTE_VECDOT
        assert np.array_equal(out.view(np.uint32), dst.view(np.uint32)), f"type {tid} {name}"
        seen.add(tid)
    assert seen == {O.Q5_0, O.Q8_0, O.Q5_K}


@pytest.mark.parametrize("ty", ["Q5_0", "Q8_0", "Q5_K"])
def test_new_type_subsums_brute_force(ty):
    """Integer partials against a float64 brute force of the dequantized blocks:
    random block bytes (finite d), random activations, the oracle's own Q8
    activation rows; sum_s block scale * partial must equal the dot of the
    dequantized values exactly (every product is an exact small integer)."""
    t = getattr(O, ty)
    rng = np.random.default_rng(7)
    qk, bs = O.BLOCK[t]
    n, rows = 512, 3
    w = rng.integers(0, 256, size=rows * (n // qk) * bs, dtype=np.uint8)
    wv = w.reshape(rows, n // qk, bs)
    # finite f16 scales: d (and dmin) in [2^-10, 2^-5)
    for off in ((0,) if qk == 32 else (0, 2)):
        e = rng.integers(0x1400, 0x2800, size=(rows, n // qk), dtype=np.uint16)
        wv[:, :, off:off + 2] = e.view(np.uint8).reshape(rows, n // qk, 2)
    x = rng.standard_normal((1, n)).astype(np.float32)
    out, route, sub = O.mul_mat(t, w, n, rows, x, 1, want_subsums=True)
    act = O.mul_mat_act(t, n, rows, x, 1)
    at = O.ACT_TYPE[t]
    aq = O.dequantize(at, act, n).astype(np.float64)
    for r in range(rows):
        wf = O.dequantize(t, w[r * O.row_size(t, n):(r + 1) * O.row_size(t, n)], n).astype(np.float64)
        ref = float(np.dot(wf, aq))
        assert abs(float(out[0, r]) - ref) <= 1e-5 * max(abs(ref), 1.0), (ty, r)
    # block sums: recompute from integer codes
    codes = act.reshape(-1)
    if qk == 32:
        aqs = np.frombuffer(codes.tobytes(), dtype=np.uint8).reshape(n // 32, 34)[:, 2:].view(np.int8).astype(np.int64)
        for r in range(rows):
            for b in range(n // 32):
                blk = wv[r, b]
                if t == O.Q8_0:
                    q = blk[2:].view(np.int8).astype(np.int64)
                else:
                    qh = int.from_bytes(bytes(blk[2:6]), "little")
                    qs = blk[6:22].astype(np.int64)
                    lo = np.concatenate([qs & 15, qs >> 4])
                    q = (lo | (((qh >> np.arange(32)) & 1) << 4)) - 16
                assert int(np.dot(q, aqs[b])) == int(sub[0, r, b]), (ty, r, b)
    else:
        # Q5_K: an integer brute force of {iacc, imin} from the raw block bytes
        # (d, dmin, 12 scale bytes, qh[32], qs[128]; 6-bit scales/mins packed as
        # in get_scale_min_k4) and the Q8_K codes; then the float64 dot of the
        # dequantized values rebuilt from the integers
        ab = np.frombuffer(codes.tobytes(), dtype=np.uint8).reshape(n // 256, 292)
        da = ab[:, :4].copy().view(np.float32).reshape(-1).astype(np.float64)
        q8 = ab[:, 4:260].copy().view(np.int8).astype(np.int64)
        for r in range(rows):
            for b in range(n // 256):
                blk = wv[r, b].astype(np.int64)
                sc8, qh, qs = blk[4:16], blk[16:48], blk[48:176]
                ia = im = 0
                for s in range(8):
                    if s < 4:
                        scl, mn = sc8[s] & 63, sc8[s + 4] & 63
                    else:
                        scl = (sc8[s + 4] & 15) | ((sc8[s - 4] >> 6) << 4)
                        mn = (sc8[s + 4] >> 4) | ((sc8[s] >> 6) << 4)
                    j = s // 2
                    nib = (qs[32 * j:32 * j + 32] >> (4 * (s & 1))) & 15
                    q5 = nib | (((qh >> s) & 1) << 4)
                    a8 = q8[b, 32 * s:32 * s + 32]
                    ia += int(scl) * int(np.dot(q5, a8))
                    im += int(mn) * int(a8.sum())
                assert (ia, im) == (int(sub[0, r, b, 0]), int(sub[0, r, b, 1])), (ty, r, b)
            d = wv[r, :, 0:2].copy().view(np.float16).reshape(-1).astype(np.float64)
            dmin = wv[r, :, 2:4].copy().view(np.float16).reshape(-1).astype(np.float64)
            ia_, im_ = sub[0, r, :, 0].astype(np.float64), sub[0, r, :, 1].astype(np.float64)
            got = float(np.sum(da * (d * ia_ - dmin * im_)))
            wf = O.dequantize(t, w[r * O.row_size(t, n):(r + 1) * O.row_size(t, n)], n).astype(np.float64)
            ref = float(np.dot(wf, aq))
            # the dequantized reference rounds d*sc and dmin*m to fp32 per element
            assert abs(got - ref) <= 1e-6 * max(abs(ref), 1.0), (r, got, ref)


def test_tiled_kquant_bit_exact():
    """tiled.rs:2183 tiled_mulmat_matches_reference_bit_exact (the Q4_K, Q5_K and
    Q6_K MUL_MAT sections)."""
    secs = fx.tiled_sections()
    assert len(secs) == 12
    for tid, n, rows, cols, xq, y, dst in secs:
        out, route, _ = O.mul_mat(tid, xq, n, rows, y, cols)
        assert route == O.ROUTE_TILED
        assert np.array_equal(out.view(np.uint32), dst.view(np.uint32)), f"type {tid} {rows}x{cols}"


def mul_mat_id_kquant(ty, xq, n, rows, ne11, n_as, n_ids, ne12, y, ids):
    """forward_mul_mat_id (compute.rs:1917-2202) for a K-quant whose experts are
    not repacked (rows % 8 != 0): every expert with >= 8 routed (slot, token)
    pairs takes the tiled kernel over its pairs in (token outer, slot inner)
    order (compute.rs:2011-2080); the other pairs take the row vec_dot.  Both
    are the oracle's MUL_MAT routes on the gathered activation rows (Q8_K from
    quantize_row_q8_K_ref in both)."""
    dst = np.zeros((ne12, n_ids, rows), dtype=np.float32)
    by_e = [[] for _ in range(n_as)]
    for t in range(ne12):
        for s in range(n_ids):
            by_e[int(ids[t, s])].append((s, t))
    for e, pairs in enumerate(by_e):
        if not pairs:
            continue
        x = np.stack([y[t, s % ne11] for s, t in pairs])
        if len(pairs) >= 8:
            out, route, _ = O.mul_mat(ty, xq[e], n, rows, x, len(pairs))
            assert route == O.ROUTE_TILED
        else:
            out = np.stack([O.mul_mat(ty, xq[e], n, rows, x[i:i + 1], 1)[0][0] for i in range(len(pairs))])
        for i, (s, t) in enumerate(pairs):
            dst[t, s] = out[i]
    return dst


def test_tiled_mul_mat_id_bit_exact():
    """tiled.rs:2205 tiled_mulmat_id_matches_reference_bit_exact for Q4_K, Q5_K and
    Q6_K experts (140 rows each, 5 experts, 4 of 16 tokens' slots routed)."""
    secs = fx.tiled_sections(kind=1)
    assert sorted(s[0] for s in secs) == [O.Q4_K, O.Q5_K, O.Q6_K]
    for tid, n, rows, ne11, n_as, n_ids, ne12, xq, y, ids, dst in secs:
        got = mul_mat_id_kquant(tid, xq, n, rows, ne11, n_as, n_ids, ne12, y, ids)
        assert np.array_equal(got.view(np.uint32), dst.view(np.uint32)), f"mmid type {tid}"


@pytest.mark.parametrize("name", fx.REAL_WEIGHT_DUMPS)
def test_real_weight_dumps_bit_exact(name):
    """vec_dot.rs:2798-2870 kquant_real_tensor_dump_vs_reference: real GGUF
    tensors through the reference's production route (the Q4_K 8x8 repack gemv
    where the tensor got the repack trait, else the row vec_dot), bit for bit,
    and the Q8_K activation bytes of the K-quants."""
    d = fx.real_weight_dump(name)
    ty, n, rows, cols = d["type"], d["n"], d["rows"], d["cols"]
    out, route, _ = O.mul_mat(ty, d["xq"], n, rows, d["act"], cols)
    assert route == (O.ROUTE_REPACK if d["flags"] & 1 else O.ROUTE_VECDOT)
    assert np.array_equal(out.view(np.uint32), d["want"].view(np.uint32)), name
    if ty in (O.Q4_K, O.Q5_K, O.Q6_K):
        q8 = np.concatenate([O.quantize(O.Q8_K, d["act"][c], kind="quantize_row_q8_K_ref") for c in range(cols)])
        assert np.array_equal(q8, d["q8k"]), name


def test_q4k_repack_dump_bit_exact():
    """repack.rs q4k_ref_tests: activation bytes, interleaved activation values,
    gemv and gemm outputs of the reference's AVX bodies."""
    d = fx.repack_dump("q4k_repack_ref.bin")
    n, nc = d["n"], d["nc"]
    assert (d["nr_gemv"], d["nr_gemm"]) == (1, 8)
    # plain q8_K rows (the gemv LHS)
    assert np.array_equal(O.quantize(O.Q8_K, d["act_g"][:n], kind="quantize_row_q8_K_ref"), d["q8"])
    # quantize_mat_q8_K_4x8: equal dequantized values d*q (sign convention may differ)
    mine = O.quantize(O.Q8_K, d["act_m"][:8 * n], kind="quantize_row_q8_K_mat")
    q8kx4 = d["q8x4"]
    for r4 in range(2):
        for r in range(4):
            row = r4 * 4 + r
            blk = mine[row * 292:(row + 1) * 292]
            dm = blk[:4].view(np.float32)[0]
            qm = blk[4:260].view(np.int8).astype(np.float32)
            t = q8kx4[r4 * 1168:(r4 + 1) * 1168]
            dr = t[4 * r:4 * r + 4].view(np.float32)[0]
            el = np.arange(256)
            qr = t[16 + (el // 8) * 32 + r * 8 + el % 8].view(np.int8).astype(np.float32)
            assert abs(dm) == abs(dr)
            assert np.array_equal((np.float32(dm) * qm).view(np.uint32), (np.float32(dr) * qr).view(np.uint32))
    # gemv (one activation row through the gemv, weights = 16 plain rows)
    out, route, _ = O.mul_mat(O.Q4_K, d["src"], n, d["nrows"], d["act_g"][:n], 1)
    assert route == O.ROUTE_REPACK
    assert np.array_equal(out[0, :nc].view(np.uint32), d["gemv"][:nc].view(np.uint32))
    # gemm (8 rows = two 4-row groups)
    out, route, _ = O.mul_mat(O.Q4_K, d["src"], n, d["nrows"], d["act_m"][:8 * n], 8)
    assert np.array_equal(out.reshape(-1).view(np.uint32), d["gemm"][:8 * nc].view(np.uint32))
    # the generic kernel really rounds differently, so the check above is sharp
    assert not np.array_equal(d["gemv"][:nc], d["gemv_gen"][:nc]) or not np.array_equal(
        d["gemm"][:8 * nc], d["gemm_gen"][:8 * nc])


def test_q4_0_repack_dump_bit_exact():
    """repack.rs q4_0_ref_tests: q8_0 activation bytes and gemv/gemm outputs."""
    d = fx.repack_dump("q4_0_repack_ref.bin")
    n, nc, nrg = d["n"], d["nc"], d["nr_gemm"]
    assert np.array_equal(O.quantize(O.Q8_0, d["act_g"][:n], kind="quantize_row_q8_0"), d["q8"])
    out, route, _ = O.mul_mat(O.Q4_0, d["src"], n, d["nrows"], d["act_g"][:n], 1)
    assert route == O.ROUTE_REPACK
    assert np.array_equal(out[0, :nc].view(np.uint32), d["gemv"][:nc].view(np.uint32))
    out, _, _ = O.mul_mat(O.Q4_0, d["src"], n, d["nrows"], d["act_m"][:nrg * n], nrg)
    assert np.array_equal(out.reshape(-1).view(np.uint32), d["gemm"][:nrg * nc].view(np.uint32))


def test_mxfp4_repack_dump_bit_exact():
    """repack.rs gemv/gemm_matches_reference_dump_bitexact (MXFP4 8x8) via the
    MUL_MAT_ID oracle with one expert and one slot."""
    d = fx.repack_dump("repack_ref.bin")
    n, nc, nrows, nrg = d["n"], d["nc"], d["nrows"], d["nr_gemm"]
    assert np.array_equal(O.quantize(O.Q8_0, d["act_g"][:n], kind="quantize_row_q8_0"), d["q8"])
    ids = np.zeros((1, 1), dtype=np.int32)
    out = O.mul_mat_id_mxfp4(d["src"], n, nrows, 1, d["act_g"][:n], 1, 1, ids, 1)
    assert np.array_equal(out.reshape(-1)[:nc].view(np.uint32), d["gemv"][:nc].view(np.uint32))
    ids = np.zeros((nrg, 1), dtype=np.int32)
    out = O.mul_mat_id_mxfp4(d["src"], n, nrows, 1, d["act_m"][:nrg * n], 1, nrg, ids, 1)
    assert np.array_equal(out.reshape(-1).view(np.uint32), d["gemm"][:nrg * nc].view(np.uint32))


def brute_q4k_subsums(wq, xq8, n):
    """Integer partials by brute force from dequantized integer parts."""
    nb = n // 256
    W = np.frombuffer(wq.tobytes(), dtype=np.uint8).reshape(-1, nb, 144)
    A = np.frombuffer(xq8.tobytes(), dtype=np.uint8).reshape(-1, nb, 292)
    out = np.zeros((A.shape[0], W.shape[0], nb, 2), dtype=np.int64)
    for r in range(W.shape[0]):
        for b in range(nb):
            blk = W[r, b]
            sc = blk[4:16]
            s = np.zeros(8, dtype=np.int64)
            m = np.zeros(8, dtype=np.int64)
            for j in range(8):
                if j < 4:
                    s[j], m[j] = sc[j] & 63, sc[j + 4] & 63
                else:
                    s[j] = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4)
                    m[j] = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4)
            qs = blk[16:144]
            nib = np.zeros(256, dtype=np.int64)
            for g in range(4):
                nib[64 * g:64 * g + 32] = qs[32 * g:32 * g + 32] & 0xF
                nib[64 * g + 32:64 * g + 64] = qs[32 * g:32 * g + 32] >> 4
            sub = np.repeat(np.arange(8), 32)
            for c in range(A.shape[0]):
                q8 = A[c, b, 4:260].view(np.int8).astype(np.int64)
                out[c, r, b, 0] = np.sum(s[sub] * nib * q8)
                out[c, r, b, 1] = np.sum(m[sub] * q8)
    return out


def test_q4k_subsums_brute_force():
    """The oracle's integer partials equal a brute-force sum, on every route."""
    rng = np.random.default_rng(7)
    n, rows = 512, 16
    w = O.quantize(O.Q4_K, (rng.standard_normal((rows, n)) * 0.02).astype(np.float32))
    for cols in (1, 5, 8):
        x = rng.standard_normal((cols, n)).astype(np.float32)
        out, route, sub = O.mul_mat(O.Q4_K, w, n, rows, x, cols, want_subsums=True)
        act = O.mul_mat_act(O.Q4_K, n, rows, x, cols)
        assert np.array_equal(sub.astype(np.int64), brute_q4k_subsums(w, act, n))
        # and the float result is the dequantized dot product within fp32 noise
        Wf = O.dequantize(O.Q4_K, w, rows * n).reshape(rows, n).astype(np.float64)
        Af = O.dequantize(O.Q8_K, act, cols * n).reshape(cols, n).astype(np.float64)
        ref = Af @ Wf.T
        assert np.max(np.abs(out - ref) / np.maximum(np.abs(ref), 1)) < 1e-5


def test_flash_attn_ref_dump_bit_exact():
    """flash_attn.rs:2195 ref_dump_bitexact: all 15 cases (one_chunk and tiled,
    F16/F32 K/V, sinks, softcap, ALiBi, DV != DK, padded KV tail)."""
    cases = fx.fa_ref_cases()
    assert len(cases) == 15
    paths = set()
    for c in cases:
        out, path = O.flash_attn_ext(c["q"], c["k"], c["v"], c["mask"], c["sinks"], c["scale"],
                                     c["max_bias"], c["softcap"])
        paths.add(path)
        assert path == (2 if c["t"] >= 64 else 3)
        assert np.array_equal(out.view(np.uint32), c["out"].view(np.uint32)), f"mode {c['mode']}"
    assert paths == {2, 3}


def test_flash_attn_probe_split_kv_bit_exact():
    """flash_attn.rs:2541 ref_probe_dump_bitexact: the T-row batch, each row
    alone and rows 1..T-1, at nth = 1 and 8 -- single rows with S_kv >= 512
    take split-KV with n_chunks = nth."""
    groups = fx.fa_probe_groups()
    n_split = 0
    for g in groups:
        for tag, ti, nth, ref in g["recs"]:
            t0, t1 = {0: (0, g["t"]), 1: (ti, ti + 1), 2: (1, g["t"])}[tag]
            q = g["q"][:, t0:t1]
            m = g["mask"][t0:t1] if g["mask"] is not None else None
            out, path = O.flash_attn_ext(q, g["k"], g["v"], m, g["sinks"], g["scale"], g["max_bias"],
                                         g["softcap"], n_chunks=nth)
            if path == 1 and nth > 1:
                n_split += 1
            assert np.array_equal(out.reshape(-1).view(np.uint32), ref.view(np.uint32)), \
                f"T={g['t']} S={g['s']} tag={tag} t={ti} nth={nth}"
    assert n_split > 0, "the probe must exercise the multi-chunk split-KV merge"


def test_flash_attn_against_float64():
    """Closed form: the oracle's three paths agree with a float64 softmax(QK^T)V
    within the f16-accumulator error, and split-KV with 1 chunk equals one_chunk."""
    rng = np.random.default_rng(2)
    H, Hkv, D = 4, 2, 64
    for T, S in [(1, 600), (3, 40), (70, 130)]:
        q = rng.standard_normal((H, T, D)).astype(np.float32)
        k = rng.standard_normal((Hkv, S, D)).astype(np.float16)
        v = rng.standard_normal((Hkv, S, D)).astype(np.float16)
        mask = np.zeros((T, S), dtype=np.float16)
        for t in range(T):
            mask[t, S - T + t + 1:] = -np.inf
        out, _ = O.flash_attn_ext(q, k, v, mask, scale=1 / 8.0, n_chunks=3)
        ref = np.zeros_like(out, dtype=np.float64)
        for h in range(H):
            kk = k[h // 2].astype(np.float64)
            vv = v[h // 2].astype(np.float64)
            s = (q[h].astype(np.float16).astype(np.float64) @ kk.T) / 8.0 + mask.astype(np.float64)
            p = np.exp(s - s.max(1, keepdims=True))
            ref[:, h] = (p / p.sum(1, keepdims=True)) @ vv
        assert np.max(np.abs(out - ref)) < 2e-3


def _q41_codes(w, ty):
    """Unsigned codes, d, m of Q4_1 / Q5_1 rows (numpy, from the block layout)."""
    bs = 20 if ty == O.Q4_1 else 24
    b = w.reshape(-1, bs)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    m = b[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
    qs = b[:, bs - 16:]
    codes = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.int64)
    if ty == O.Q5_1:
        qh = b[:, 4:8].copy().view(np.uint32)[:, 0].astype(np.int64)
        codes |= ((qh[:, None] >> np.arange(32)) & 1) << 4
    return codes, d, m


@pytest.mark.parametrize("ty", [O.Q4_1, O.Q5_1])
def test_q41_q51_vec_dot_brute_force(ty):
    """vec_dot_q4_1_q8_1 / vec_dot_q5_1_q8_1 (no reference fixture holds their
    dots): the exact integer block sums from numpy, and the float result
    against sum_b d*d8*isum_b + m*s_b in float64 (the reference's formula, only
    the fp32 summation order open); quantized rows from the pinned quantizers,
    plus random block bytes with the top codes."""
    rng = np.random.default_rng(5)
    n = 1024
    for trial in range(6):
        if trial < 3:
            w = O.quantize(ty, rng.standard_normal(n).astype(np.float32) * 0.1)
        else:
            bs = 20 if ty == O.Q4_1 else 24
            w = rng.integers(0, 256, size=n // 32 * bs, dtype=np.uint8)
            blk = w.reshape(-1, bs)
            blk[:, 0:2] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
            blk[:, 2:4] = np.frombuffer(np.float16(-0.3).tobytes(), np.uint8)
        x = rng.standard_normal(n).astype(np.float32) * (10.0 if trial == 2 else 1.0)
        a = O.quantize(O.Q8_1, x)
        ab = a.reshape(-1, 36)
        d8 = ab[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
        s8 = ab[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
        q8 = ab[:, 4:].view(np.int8).astype(np.int64)
        assert np.all(np.abs(s8 - np.float16(d8 * q8.sum(1)).astype(np.float64)) <= 1e-3 * np.abs(s8) + 1e-7)
        codes, d, m = _q41_codes(w, ty)
        isum = (codes * q8).sum(1)
        want = float(np.sum(d * d8 * isum + m * s8))
        f = O.lib().oracle_vec_dot_q4_1_q8_1 if ty == O.Q4_1 else O.lib().oracle_vec_dot_q5_1_q8_1
        got = f(n, O._p(np.ascontiguousarray(w)), O._p(a))
        scale = float(np.sum(np.abs(d * d8 * isum)) + np.sum(np.abs(m * s8)))
        assert abs(got - want) <= 1e-6 * scale, (trial, got, want)
        # the routed MUL_MAT exports the same integer block sums
        out, route, sub = O.mul_mat(ty, w, n, 1, x[None, :], 1, want_subsums=True)
        assert route == O.ROUTE_VECDOT
        assert np.array_equal(sub.reshape(-1), isum)
        assert out[0, 0] == np.float32(got)


def test_q2k_q3k_dequant_bit_exact():
    """quants_ref.bin sections 10 (Q2_K) and 11 (Q3_K): the oracle's
    dequantize_row of the reference's bytes equals the reference's values."""
    secs = {tid: (q, deq) for (_, tid, n, q, deq) in fx.quant_sections("quants_ref.bin")}
    for tid in (O.Q2_K, O.Q3_K):
        q, deq = secs[tid]
        assert deq.any()
        got = O.dequantize(tid, q, 1024)
        assert np.array_equal(got.view(np.uint32), deq.view(np.uint32)), f"type {tid}"


def _k23_terms(w, ty, act, n):
    """numpy brute force per super-block: (isum, summs, d, dmin) from the block
    bytes (Q2_K: 4-bit scale | 4-bit min; Q3_K: 6-bit scales - 32, 3-bit codes)"""
    nb = n // 256
    a = act.reshape(nb, 292)
    d8 = a[:, 0:4].copy().view(np.float32)[:, 0].astype(np.float64)
    q8 = a[:, 4:260].view(np.int8).astype(np.int64)
    bs = a[:, 260:292].copy().view(np.int16).astype(np.int64)
    deq = O.dequantize(ty, w, n).reshape(nb, 256).astype(np.float64)
    if ty == O.Q2_K:
        b = w.reshape(nb, 84)
        sc = b[:, 0:16].astype(np.int64)
        qs = b[:, 16:80]
        d = b[:, 80:82].copy().view(np.float16)[:, 0].astype(np.float64)
        dm = b[:, 82:84].copy().view(np.float16)[:, 0].astype(np.float64)
        # code of element 128j + 32k + e: (qs[32j + e] >> 2k) & 3
        codes = np.zeros((nb, 256), np.int64)
        for j in range(2):
            for k in range(4):
                codes[:, 128 * j + 32 * k:128 * j + 32 * k + 32] = (qs[:, 32 * j:32 * j + 32] >> (2 * k)) & 3
        g = (codes * q8).reshape(nb, 16, 16).sum(-1)
        isum = ((sc & 15) * g).sum(-1)
        summs = ((sc >> 4) * bs).sum(-1)
        # the dequantized values agree with the codes / scales read here
        want_deq = np.repeat(d[:, None] * (sc & 15), 16, 1) * codes - np.repeat(dm[:, None] * (sc >> 4), 16, 1)
        assert np.allclose(deq, want_deq, rtol=1e-6, atol=1e-30)
        return isum, summs, d8 * d, d8 * dm
    b = w.reshape(nb, 110)
    d = b[:, 108:110].copy().view(np.float16)[:, 0].astype(np.float64)
    # values from the pinned dequantizer: v * (sc - 32) * d, integers once divided back
    scale_vals = np.zeros((nb, 16), np.float64)
    codes = np.zeros((nb, 256), np.int64)
    hm = b[:, 0:32]
    qs = b[:, 32:96]
    for j in range(2):
        for k in range(4):
            lo = ((qs[:, 32 * j:32 * j + 32] >> (2 * k)) & 3).astype(np.int64)
            hb = (hm >> (4 * j + k)) & 1
            codes[:, 128 * j + 32 * k:128 * j + 32 * k + 32] = np.where(hb != 0, lo, lo - 4)
    raw = b[:, 96:108]
    aux = raw.copy().view(np.uint32).astype(np.uint64)
    km1, km2 = 0x03030303, 0x0f0f0f0f
    w4 = [(aux[:, 0] & km2) | ((aux[:, 2] & km1) << 4), (aux[:, 1] & km2) | (((aux[:, 2] >> 2) & km1) << 4),
          ((aux[:, 0] >> 4) & km2) | (((aux[:, 2] >> 4) & km1) << 4),
          ((aux[:, 1] >> 4) & km2) | (((aux[:, 2] >> 6) & km1) << 4)]
    for i in range(16):
        scale_vals[:, i] = ((w4[i >> 2] >> (8 * (i & 3))) & 0xff).astype(np.float64) - 32
    g = (codes * q8).reshape(nb, 16, 16).sum(-1)
    isum = (scale_vals.astype(np.int64) * g).sum(-1)
    want_deq = np.repeat(d[:, None] * scale_vals, 16, 1) * codes
    assert np.allclose(deq, want_deq, rtol=1e-6, atol=1e-30)
    return isum, np.zeros(nb, np.int64), d8 * d, np.zeros(nb)


@pytest.mark.parametrize("ty", [O.Q2_K, O.Q3_K])
def test_q2k_q3k_vec_dot_brute_force(ty):
    """vec_dot_q2_K_q8_K / vec_dot_q3_K_q8_K (no reference fixture holds their
    dots): exact integer sums from numpy on the block bytes (the value layout
    itself checked against the fixture-pinned dequantizer), the float result
    against sum d8*d*isum - d8*dmin*summs in float64, and the routed MUL_MAT's
    integer exports; the reference's own quantized bytes (quants_ref.bin) and
    random blocks."""
    rng = np.random.default_rng(21)
    secs = {tid: q for (_, tid, n, q, deq) in fx.quant_sections("quants_ref.bin")}
    bs = 84 if ty == O.Q2_K else 110
    for trial in range(5):
        if trial == 0:
            w, n = np.ascontiguousarray(secs[ty]), 1024
        else:
            n = 1024
            w = rng.integers(0, 256, size=(n // 256) * bs, dtype=np.uint8)
            blk = w.reshape(-1, bs)
            off = 80 if ty == O.Q2_K else 108
            blk[:, off:off + 2] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
            if ty == O.Q2_K:
                blk[:, 82:84] = np.frombuffer(np.float16(0.02).tobytes(), np.uint8)
        x = rng.standard_normal(n).astype(np.float32) * (5.0 if trial == 2 else 1.0)
        a = O.quantize(O.Q8_K, x, kind="quantize_row_q8_K_ref")
        isum, summs, dd, dmn = _k23_terms(w, ty, a, n)
        want = float(np.sum(dd * isum - dmn * summs))
        f = O.lib().oracle_vec_dot_q2_K_q8_K if ty == O.Q2_K else O.lib().oracle_vec_dot_q3_K_q8_K
        got = f(n, O._p(np.ascontiguousarray(w)), O._p(a))
        scale = float(np.sum(np.abs(dd * isum)) + np.sum(np.abs(dmn * summs)))
        assert abs(got - want) <= 1e-6 * scale, (trial, got, want)
        out, route, sub = O.mul_mat(ty, w, n, 1, x[None, :], 1, want_subsums=True)
        assert route == O.ROUTE_VECDOT
        if ty == O.Q2_K:
            assert np.array_equal(sub.reshape(-1, 2)[:, 0], isum) and np.array_equal(sub.reshape(-1, 2)[:, 1], summs)
        else:
            assert np.array_equal(sub.reshape(-1), isum)
        assert out[0, 0] == np.float32(got)


VD3 = {O.IQ4_NL: "vec_dot_iq4_nl_q8_0", O.IQ4_XS: "vec_dot_iq4_xs_q8_K", O.NVFP4: "vec_dot_nvfp4_q8_0"}


@pytest.mark.parametrize("ty", sorted(VD3))
def test_vecdot3_bit_exact(ty):
    """vec_dot.rs vecdot3 ground truth (parity/ref_vecdot_dump3.c): the x86
    kernels of NVFP4, IQ4_NL and IQ4_XS on LCG block bytes and the reference's
    own quantized activations; the oracle's fp32 order reproduces the result
    bit for bit."""
    (sec,) = [s for s in fx.vecdot3_sections() if s[0] == ty]
    _, n, xq, yq, want = sec
    got = np.float32(getattr(O.lib(), "oracle_" + VD3[ty])(n, O._p(xq), O._p(yq)))
    assert got.view(np.uint32) == want.view(np.uint32), (got, want)


def test_vecdot3_dot_is_the_brute_force_of_the_dequantized_rows():
    """What fixes the dots beyond the dumped fp32 results: each equals, to fp32
    rounding, the float64 dot of the dequantized weights with the dequantized
    activations (a dropped term, a wrong nibble order or scale would not)."""
    for ty, name in VD3.items():
        (sec,) = [s for s in fx.vecdot3_sections() if s[0] == ty]
        _, n, xq, yq, want = sec
        w = O.dequantize(ty, xq, n).astype(np.float64)
        a = O.dequantize(O.ACT_TYPE[ty], yq, n).astype(np.float64) if O.ACT_TYPE[ty] == O.Q8_0 else None
        if a is None:  # Q8_K rows: codes * d per 256-block
            a = np.concatenate([np.frombuffer(yq[i * 292 + 4:i * 292 + 260].tobytes(), np.int8).astype(np.float64) *
                                np.frombuffer(yq[i * 292:i * 292 + 4].tobytes(), np.float32)[0] for i in range(n // 256)])
        exact = float(np.dot(w, a))
        assert abs(float(want) - exact) <= 1e-5 * max(1.0, np.abs(w * a).sum()), (ty, want, exact)


@pytest.mark.parametrize("ty", [O.IQ4_NL, O.IQ4_XS])
def test_iq4_dequant_bit_exact(ty):
    """quants_k.rs iq dequant parity (parity/ref_quants_dump.c, quants_ref_iq.bin):
    the reference quantizer's IQ4_NL / IQ4_XS bytes dequantize to the dumped
    floats bit for bit."""
    (sec,) = [s for s in fx.quant_sections("quants_ref_iq.bin") if s[1] == ty]
    _, _, n, q, deq = sec
    got = O.dequantize(ty, q, n)
    assert np.array_equal(got.view(np.uint32), deq.view(np.uint32))


def test_nvfp4_dequant_and_ue4m3():
    """quants.rs fp4_dequant_bit_exact_vs_reference for NVFP4 (quants_ref_fp4.bin)
    and the UE4M3 closed form over all 256 bytes: 0 for 0x00 and 0x7F,
    man * 2^-10 for exp 0, (8 + man) * 2^(exp - 11) otherwise."""
    secs = [s for s in fx.quant_sections("quants_ref_fp4.bin") if s[1] == O.NVFP4]
    assert len(secs) == 4
    for magic, tid, n, q, deq in secs:
        got = O.dequantize(O.NVFP4, q, n)
        assert np.array_equal(got.view(np.uint32), deq.view(np.uint32))
    L = O.lib()
    for x in range(256):
        e, m = (x >> 3) & 15, x & 7
        want = 0.0 if x in (0, 0x7F) else (m * 2.0 ** -10 if e == 0 else (8 + m) * 2.0 ** (e - 11))
        assert np.float32(L.oracle_ue4m3_to_fp32(x)) == np.float32(want), x


def test_tiled_k23_iq4xs_bit_exact():
    """tiled.rs:2183 tiled_mulmat_matches_reference_bit_exact for Q2_K, Q3_K and
    IQ4_XS (parity/tiled_ref.bin, the sections kept in tiled_ref_k23x.bin): from
    8 columns the oracle folds each super-block's exact sums as the tiled
    kernel's epilogue does, bit for bit; below 8 it is the row vec_dot."""
    secs = fx.tiled_sections("tiled_ref_k23x.bin")
    assert sorted({s[0] for s in secs}) == [O.Q2_K, O.Q3_K, O.IQ4_XS]
    for tid, n, rows, cols, xq, y, dst in secs:
        got, route, _ = O.mul_mat(tid, xq, n, rows, y, cols)
        want_route = O.ROUTE_TILED if cols >= 8 else O.ROUTE_VECDOT
        assert route == want_route
        if route == O.ROUTE_TILED:
            assert np.array_equal(got.view(np.uint32), dst.reshape(cols, rows).view(np.uint32)), (tid, rows, cols)


@pytest.mark.parametrize("ty,name", [(O.Q1_0, "vec_dot_q1_0_q8_0"), (O.Q2_0, "vec_dot_q2_0_q8_0")])
def test_q1_q2_vecdot_bit_exact(ty, name):
    """vecdot3_ref.bin types 41 / 42 (vec_dot.rs:1074, :1120): bit for bit."""
    (sec,) = [s for s in fx.vecdot3_sections() if s[0] == ty]
    _, n, xq, yq, want = sec
    got = np.float32(getattr(O.lib(), "oracle_" + name)(n, O._p(xq), O._p(yq)))
    assert got.view(np.uint32) == want.view(np.uint32), (got, want)


@pytest.mark.parametrize("ty", [O.Q1_0, O.Q2_0])
def test_q1_q2_quantizer_and_dequant_bit_exact(ty):
    """quants.rs q1_0 / q2_0 parity (parity/ref_quants_dump.c,
    quants_ref_q1q2.bin): the quantizers' bytes and the dequantized floats."""
    secs = [s for s in fx.quant_sections("quants_ref_q1q2.bin") if s[1] == ty]
    assert secs
    for magic, tid, n, q, deq in secs:
        x = fx.ref_input(n)
        assert np.array_equal(O.quantize(ty, x), q)
        got = O.dequantize(ty, q, n)
        assert np.array_equal(got.view(np.uint32), deq.view(np.uint32))


def test_bf16_conversion_against_torch():
    """the oracle's f32 -> bf16 (half's RNE) against torch's bfloat16 cast on
    ties, subnormals, infinities and random bit patterns"""
    import torch
    rng = np.random.default_rng(3)
    bits = np.concatenate([rng.integers(0, 2 ** 32, size=20000, dtype=np.uint64).astype(np.uint32),
                           np.array([0x3f808000, 0x3f818000, 0x00008000, 0x00018000, 0x7f7fffff, 0x7f800000,
                                     0xff800000, 0x80000000, 0x00000001, 0x7f7f8000], dtype=np.uint32)])
    f = bits.view(np.float32)
    fin = np.isfinite(f)
    want = torch.from_numpy(f[fin].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([O.fp32_to_bf16(v) for v in f[fin]], dtype=np.uint16)
    assert np.array_equal(got, want)
    nan = np.array([O.fp32_to_bf16(v) for v in f[~np.isfinite(f) & np.isnan(f)]], dtype=np.uint16)
    assert np.all((nan & 0x7f80) == 0x7f80) and np.all(nan & 0x007f)


@pytest.mark.parametrize("ty", [O.F32, O.F16, O.BF16])
def test_dense_mul_mat_brute_force(ty):
    """F32 / F16 / BF16 MUL_MAT: activations rounded to the weight type (numpy
    float16 / torch bfloat16 casts), products in f32, summed in float64"""
    import torch
    rng = np.random.default_rng(ty + 5)
    n, rows, cols = 1000, 7, 3
    wf = rng.standard_normal((rows, n)).astype(np.float32)
    x = rng.standard_normal((cols, n)).astype(np.float32)
    if ty == O.F32:
        w, wv, xv = wf, wf, x
    elif ty == O.F16:
        w = wf.astype(np.float16).view(np.uint16)
        wv, xv = wf.astype(np.float16).astype(np.float32), x.astype(np.float16).astype(np.float32)
    else:
        w = torch.from_numpy(wf).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        wv = torch.from_numpy(wf).to(torch.bfloat16).float().numpy()
        xv = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    prod = (wv[None, :, :] * xv[:, None, :]).astype(np.float32).astype(np.float64)
    want = prod.sum(-1).astype(np.float32)
    got = O.mul_mat_dense(ty, w, n, rows, x, cols)
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1)) <= 1e-6


@pytest.mark.parametrize("ty", [O.IQ2_XXS, O.IQ2_XS, O.IQ2_S, O.IQ3_XXS, O.IQ3_S, O.IQ1_S, O.IQ1_M])
def test_iq_grid_vecdot_bit_exact(ty):
    """vecdot3_ref.bin's IQ1 / IQ2 / IQ3 sections (the reference's x86 dots on
    its block bytes and quantized activation row): bit for bit.  The grids,
    sign parity, scale nibbles, qh bits and deltas all enter these."""
    (sec,) = [s for s in fx.vecdot3_sections() if s[0] == ty]
    _, n, xq, yq, want = sec
    got = O.vec_dot_iq(ty, n, xq, yq)
    assert got.view(np.uint32) == want.view(np.uint32), (got, want)


@pytest.mark.parametrize("ty", [O.IQ2_XXS, O.IQ2_XS, O.IQ2_S, O.IQ3_XXS, O.IQ3_S, O.IQ1_S, O.IQ1_M])
def test_iq_grid_tiled_sections(ty):
    """tiled_ref_iq.bin (the reference's tiled kernel, tiled.rs:2183, 8+
    columns): the oracle's tiled fold of the exact super-block integers
    reproduces the dumped outputs bit for bit."""
    secs = [s for s in fx.tiled_sections("tiled_ref_iq.bin") if s[0] == ty]
    assert secs
    for tid, n, rows, cols, xq, y, dst in secs:
        got, route, _ = O.mul_mat(tid, xq.reshape(rows, -1), n, rows, y, cols)
        assert route == O.ROUTE_TILED
        assert np.array_equal(got.reshape(dst.shape).view(np.uint32), dst.view(np.uint32))
