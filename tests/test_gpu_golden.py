"""The reference's own golden vectors computed on the GPU.

  * real GGUF tensors x the reference's production route
    (parity/{q4k_goss,q4k_granite,q6k_granite,q5_0_goss,q8_0_goss,q5k_real}_ref.bin,
    vec_dot.rs:2798-2870): the GPU output at the dump's own column count and
    for its first column alone, within 1e-5 by rel_err (vec_dot.rs:2355), and
    the Q8_K activation bytes bit for bit;
  * the tiled MUL_MAT sections of parity/tiled_ref.bin (tiled.rs:2183; Q4_K,
    Q5_K, Q6_K; 12-300 weight rows that are not multiples of 8, 8-300
    activation rows): the Q4_K GEMM with N % 8 != 0 on reference-quantized
    activations, the Q6_K GEMM and the 8-column decode kernels, activation
    bytes bit for bit; fp32 within the reference's own route-to-route gap on
    these inputs (see test_tiled_sections);
  * parity/fa_ref.bin (flash_attn.rs:2064-2117) and fa_probe.bin
    (flash_attn.rs:2541-2640): every case within 2e-3 max-abs (f16 and f32
    K/V, DK != DV, head sizes 16 / 32 / 64).
The oracle is pinned bit-exact on the same files (test_oracle_golden.py).
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


def rel_err(a, b):
    return float(np.max(np.abs(a - b) / np.maximum(np.abs(b), 1.0))) if a.size else 0.0


@pytest.mark.parametrize("name", fx.REAL_WEIGHT_DUMPS)
def test_real_weight_dumps(be, name):
    d = fx.real_weight_dump(name)
    ty, n, rows, cols = d["type"], d["n"], d["rows"], d["cols"]
    print(f"dump {name} type={ty} n={n} rows={rows} cols={cols}", flush=True)
    wd = torch.from_numpy(d["xq"].reshape(rows, -1)).cuda()
    xd = torch.from_numpy(np.ascontiguousarray(d["act"])).cuda()
    got = be.mul_mat(wd, ty, n, xd).cpu().numpy()
    assert rel_err(got, d["want"]) <= 1e-5, rel_err(got, d["want"])
    one = be.mul_mat(wd, ty, n, xd[:1].contiguous()).cpu().numpy()
    assert rel_err(one, d["want"][:1]) <= 1e-5
    if ty in (O.Q4_K, O.Q5_K, O.Q6_K):
        act = be.mul_mat_act(wd, ty, n, xd).cpu().numpy().reshape(-1)
        assert np.array_equal(act, d["q8k"])


@pytest.mark.parametrize("idx", range(12))
def test_tiled_sections(be, idx):
    """These dumps hold outputs up to ~7e3 built from terms that cancel
    (random block bytes): the reference's own two routes for them (the row
    vec_dot and the tiled kernel) differ by 1e-5 .. 8.7e-4 in rel_err.  The GPU
    keeps the exact integers and folds them in its own fp32 order, so its bar
    here is that route-to-route gap of the reference itself (1e-5 at least),
    and the normwise error stays below 1e-6."""
    tid, n, rows, cols, xq, y, dst = fx.tiled_sections()[idx]
    print(f"tiled type={tid} n={n} rows={rows} cols={cols}", flush=True)
    wd = torch.from_numpy(xq.reshape(rows, -1)).cuda()
    xd = torch.from_numpy(np.ascontiguousarray(y)).cuda()
    got = be.mul_mat(wd, tid, n, xd).cpu().numpy()
    vec_dot = np.concatenate([O.mul_mat(tid, xq, n, rows, y[c:c + 1], 1)[0] for c in range(cols)])
    gap = rel_err(vec_dot, dst)
    err = rel_err(got, dst)
    print(f"  rel_err {err:.2e}; reference vec_dot vs tiled {gap:.2e}", flush=True)
    assert err <= max(1e-5, gap), (err, gap)
    assert np.linalg.norm(got - dst) <= 1e-6 * np.linalg.norm(dst)
    act = be.mul_mat_act(wd, tid, n, xd).cpu().numpy().reshape(-1)
    assert np.array_equal(act, O.mul_mat_act(tid, n, rows, y, cols))


def fa_run(be, q, k, v, mask, sinks, scale, max_bias, softcap):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda() if a is not None else None
    return be.flash_attn_ext(t(q), t(k), t(v), t(mask), t(sinks), scale, max_bias, softcap).cpu().numpy()


def test_fa_ref_cases(be):
    """Every case of the reference's table: f16 and f32 K/V, DK != DV, head
    sizes 16 / 32 / 64, GQA up to 8, masks, sinks, softcap, ALiBi."""
    cases = fx.fa_ref_cases()
    assert len(cases) == 15
    for i, c in enumerate(cases):
        print(f"fa_ref case {i} mode={c['mode']} dk={c['dk']} dv={c['dv']} h={c['h']}/{c['h_kv']} "
              f"t={c['t']} s={c['s']} kv={c['k'].dtype}", flush=True)
        args = (c["q"], c["k"], c["v"], c["mask"], c["sinks"], c["scale"], c["max_bias"], c["softcap"])
        got = fa_run(be, *args)
        err = float(np.max(np.abs(got - c["out"])))
        assert err <= 2e-3, (i, err)


def test_fa_probe(be):
    """fa_probe.bin: the T-row batch (tag 0), each row alone (tag 1, the
    split-KV decode route at S = 600) and rows 1..T-1 (tag 2)."""
    for g in fx.fa_probe_groups():
        args = (g["scale"], g["max_bias"], g["softcap"])
        for tag, ti, nth, out in g["recs"]:
            if tag == 0:
                q, mask = g["q"], g["mask"]
            elif tag == 1:
                q, mask = g["q"][:, ti:ti + 1], None if g["mask"] is None else g["mask"][ti:ti + 1]
            else:
                q, mask = g["q"][:, 1:], None if g["mask"] is None else g["mask"][1:]
            print(f"fa_probe tag={tag} t={ti} T={q.shape[1]} S={g['s']}", flush=True)
            got = fa_run(be, q, g["k"], g["v"], mask, g["sinks"], *args)
            err = float(np.max(np.abs(got.reshape(-1) - out)))
            assert err <= 2e-3, (tag, ti, err)
