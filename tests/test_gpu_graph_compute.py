"""GPU tests of ghip_graph_compute (BackendI.graph_compute, backend.rs:652-668):
a node list computed in order, with consecutive sibling MUL_MATs (one f32
activation row, same src1, same K-quant type and K) in one launch.

The bar: every node's output bit-identical to the single-op entry point
(whose own parity with the oracle is tested elsewhere), plus oracle parity
of grouped nodes on ragged shapes at the MUL_MAT bar (fp32 within 1e-5 by
rel_err = max |a-b| / max(|b|, 1), vec_dot.rs:2355).
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


def weights(be, ty, n, k, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return be.quantize(torch.randn((n, k), device="cuda", generator=g) * 0.02, ty)


@pytest.mark.parametrize("ty,m", [(12, 1), (12, 2), (12, 3), (12, 4), (12, 5), (12, 8), (14, 1), (14, 2), (2, 1), (2, 2),
                                  (2, 4)])
def test_decode_layer_groups_bit_identical(be, ty, m):
    """q/k/v (4096 -> 4096, 1024, 1024) and gate/up (4096 -> 14336) as two
    groups, o as a single node, at m activation rows (Q4_K, Q6_K, Q4_0; Q5_K,
    Q5_0 and Q8_0 groups are in the ragged test): every output equals
    ghip_mul_mat's."""
    import ghip
    k = 4096
    shapes = [("q", 4096), ("k", 1024), ("v", 1024), ("o", 4096), ("gate", 14336), ("up", 14336)]
    ws = {name: weights(be, ty, n, k, i) for i, (name, n) in enumerate(shapes)}
    g = torch.Generator(device="cuda").manual_seed(99)
    x = torch.randn((m, k), device="cuda", generator=g)
    xo = torch.randn((m, k), device="cuda", generator=g)  # o reads another activation
    outs = {name: torch.full((m, n), float("nan"), device="cuda") for name, n in shapes}
    nodes = [ghip.mul_mat_node(ws[nm], ty, k, xo if nm == "o" else x, outs[nm]) for nm, _ in shapes]
    be.graph_compute(nodes)
    torch.cuda.synchronize()
    for nm, _ in shapes:
        ref = be.mul_mat(ws[nm], ty, k, xo if nm == "o" else x)
        torch.cuda.synchronize()
        assert torch.equal(outs[nm], ref), nm


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8])
def test_mixed_row_counts_bit_identical(be, m):
    """Siblings on both sides of the 8192-row line (4096 and 14336 rows, in
    both orders): a single op picks its decode kernel by its own row count,
    so a group must never run a member on a kernel its single op would not
    use; every output equals ghip_mul_mat's."""
    import ghip
    k = 4096
    for order in ((4096, 14336, 1024), (14336, 4096, 1024)):
        ws = [weights(be, 12, n, k, 20 + i) for i, n in enumerate(order)]
        g = torch.Generator(device="cuda").manual_seed(m)
        x = torch.randn((m, k), device="cuda", generator=g)
        outs = [torch.full((m, n), float("nan"), device="cuda") for n in order]
        be.graph_compute([ghip.mul_mat_node(w, 12, k, x, o) for w, o in zip(ws, outs)])
        torch.cuda.synchronize()
        for w, o, n in zip(ws, outs, order):
            ref = be.mul_mat(w, 12, k, x)
            torch.cuda.synchronize()
            assert torch.equal(o, ref), (order, n)


@pytest.mark.parametrize("ty,k,ns,m", [(12, 1024, (96, 40, 8), 1), (13, 768, (33, 64), 1), (14, 512, (17, 31, 64, 5), 1),
                                       (12, 512, (96, 40, 8), 3), (13, 512, (24, 40, 8), 6),
                                       (12, 512, (36, 40, 64, 20), 4),  # N % 8 differs: two groups
                                       (2, 1024, (64, 40, 8), 1), (2, 512, (64, 40, 8), 3), (6, 512, (48, 16), 3),
                                       (8, 768, (24, 40, 8, 16), 5), (6, 1024, (100, 36), 1)])
def test_group_ragged_vs_oracle(be, ty, k, ns, m):
    """groups whose matrices end inside a workgroup's rows, at m activation
    rows, against the oracle"""
    import ghip
    rng = np.random.default_rng(7)
    wf = [(rng.standard_normal((n, k)) * 0.02).astype(np.float32) for n in ns]
    x = rng.standard_normal((m, k)).astype(np.float32)
    wq = [O.quantize(ty, w).reshape(w.shape[0], -1) for w in wf]
    wd = [torch.from_numpy(q).cuda() for q in wq]
    xd = torch.from_numpy(x).cuda()
    outs = [torch.full((m, n), float("nan"), device="cuda") for n in ns]
    be.graph_compute([ghip.mul_mat_node(w, ty, k, xd, o) for w, o in zip(wd, outs)])
    torch.cuda.synchronize()
    for q, w, n, o in zip(wq, wd, ns, outs):
        ref, _, _ = O.mul_mat(ty, q, k, n, x, m)
        got = o.cpu().numpy()
        assert np.isfinite(got).all()
        assert rel_err(got, ref) <= TOL
        single = be.mul_mat(w, ty, k, xd)
        torch.cuda.synchronize()
        assert torch.equal(o, single)


@pytest.mark.parametrize("m,k,ns", [(16, 1024, (512, 128, 128)), (100, 768, (200, 64, 72)), (512, 1024, (256, 256))])
def test_prefill_group_vs_oracle(be, m, k, ns):
    """Q4_K siblings at prefill batches run as one GEMM launch (one Q8_K
    quantization and layout for all): every member against the oracle at the
    MUL_MAT bar, and against its single-op call within the same bar (alone,
    a small matrix takes the split-K route, whose ordered slice sums round
    differently)."""
    import ghip
    rng = np.random.default_rng(11)
    wf = [(rng.standard_normal((n, k)) * 0.02).astype(np.float32) for n in ns]
    x = rng.standard_normal((m, k)).astype(np.float32)
    wq = [O.quantize(12, w).reshape(w.shape[0], -1) for w in wf]
    wd = [torch.from_numpy(q).cuda() for q in wq]
    xd = torch.from_numpy(x).cuda()
    outs = [torch.full((m, n), float("nan"), device="cuda") for n in ns]
    be.graph_compute([ghip.mul_mat_node(w, 12, k, xd, o) for w, o in zip(wd, outs)])
    torch.cuda.synchronize()
    for q, w, n, o in zip(wq, wd, ns, outs):
        ref, _, _ = O.mul_mat(12, q, k, n, x, m)
        got = o.cpu().numpy()
        assert np.isfinite(got).all()
        assert rel_err(got, ref) <= TOL
        single = be.mul_mat(w, 12, k, xd).cpu().numpy()
        assert rel_err(got, single) <= TOL


def test_dependent_and_aliased_nodes_keep_order(be):
    """a node reading its predecessor's dst, and two nodes writing the same
    dst, are not grouped: the graph computes them in order"""
    import ghip
    k = 1024
    w1, w2, w3 = (weights(be, 12, 1024, k, s) for s in (1, 2, 3))
    x = torch.randn((1, k), device="cuda")
    y1 = torch.empty((1, 1024), device="cuda")
    y2 = torch.empty((1, 1024), device="cuda")
    shared = torch.empty((1, 1024), device="cuda")
    nodes = [ghip.mul_mat_node(w1, 12, k, x, y1),
             ghip.mul_mat_node(w2, 12, k, y1, y2),      # reads node 0's output
             ghip.mul_mat_node(w1, 12, k, x, shared),
             ghip.mul_mat_node(w3, 12, k, x, shared)]   # overwrites node 2's dst
    be.graph_compute(nodes)
    torch.cuda.synchronize()
    r1 = be.mul_mat(w1, 12, k, x)
    r2 = be.mul_mat(w2, 12, k, r1)
    r3 = be.mul_mat(w3, 12, k, x)
    torch.cuda.synchronize()
    assert torch.equal(y1, r1) and torch.equal(y2, r2) and torch.equal(shared, r3)


def test_mixed_ops_and_fusion_switch(be, monkeypatch):
    """MUL_MAT, MUL_MAT_ID and FLASH_ATTN_EXT nodes in one list equal the
    single-op calls, with the grouping on and off"""
    import ghip
    k = 2880
    wa = weights(be, 12, 512, 1024, 4)
    wb = weights(be, 12, 256, 1024, 5)
    x = torch.randn((1, 1024), device="cuda")
    experts = be.quantize(torch.randn((4 * 64, k), device="cuda") * 0.02, ghip.MXFP4).view(4, 64, -1)
    b = torch.randn((3, 1, k), device="cuda")
    ids = torch.tensor([[0, 3], [2, 1], [3, 3]], dtype=torch.int32, device="cuda")
    H, T, D, S = 4, 2, 64, 300
    q = torch.randn((H, T, D), device="cuda")
    kk = torch.randn((2, S, D), device="cuda").half()
    vv = torch.randn((2, S, D), device="cuda").half()
    refs = [be.mul_mat(wa, 12, 1024, x), be.mul_mat(wb, 12, 1024, x), be.mul_mat_id(experts, k, b, ids),
            be.flash_attn_ext(q, kk, vv, None, None, 0.125)]
    torch.cuda.synchronize()
    for fuse in ("1", "0"):
        monkeypatch.setenv("GHIP_GRAPH_FUSE", fuse)
        outs = [torch.empty_like(r) for r in refs]
        nodes = [ghip.mul_mat_node(wa, 12, 1024, x, outs[0]), ghip.mul_mat_node(wb, 12, 1024, x, outs[1]),
                 ghip.mul_mat_id_node(experts, k, b, ids, outs[2]),
                 ghip.flash_attn_node(q, kk, vv, None, None, outs[3], scale=0.125)]
        be.graph_compute(nodes)
        torch.cuda.synchronize()
        for o, r in zip(outs, refs):
            assert torch.equal(o, r), fuse


def test_errors(be):
    import ghip
    be.graph_compute([])  # nothing to do
    bad = ghip.Node(99, [], None)
    with pytest.raises(ghip.GhipError, match="op 99 not supported"):
        be.graph_compute([bad])
    # a failing node reports its own error (TQ1_0 weights are refused, as the
    # reference refuses them: compute.rs:1456-1464)
    ghip.BLOCK.setdefault(34, (256, 54))
    w = torch.zeros((32, 54), dtype=torch.uint8, device="cuda")
    x = torch.randn((1, 256), device="cuda")
    out = torch.empty((1, 32), device="cuda")
    node = ghip.Node(ghip.OP_MUL_MAT, [ghip.describe(w, 34, 256), ghip.describe(x, ghip.F32)], ghip.describe(out, ghip.F32))
    with pytest.raises(ghip.GhipError, match="not supported"):
        be.graph_compute([node])


@pytest.mark.parametrize("m", [4, 8])
def test_prequantized_inputs(be, monkeypatch, m):
    """The whole-K decode groups whose activation rows no earlier node writes
    are quantized in one launch before the first node; a node reading an
    earlier node's output (down after gate) is quantized in order.  Every
    output equals the result without the pre-pass (GHIP_GRAPH_PREQUANT=0)
    and ghip_mul_mat's."""
    import ghip
    k = 4096
    g = torch.Generator(device="cuda").manual_seed(m + 50)
    shapes = [("q", 12, k, 4096), ("k", 12, k, 1024), ("v", 12, k, 1024), ("o", 12, k, 4096),
              ("gate", 12, k, 14336), ("down", 14, 14336, 4096)]
    ws = {nm: weights(be, ty, n, kk, i + 30) for i, (nm, ty, kk, n) in enumerate(shapes)}
    x = torch.randn((m, k), device="cuda", generator=g)
    xo = torch.randn((m, k), device="cuda", generator=g)
    print(f"prequantized inputs m={m}", flush=True)

    def run():
        outs = {nm: torch.full((m, n), float("nan"), device="cuda") for nm, _, _, n in shapes}
        src = {"q": x, "k": x, "v": x, "o": xo, "gate": x, "down": outs["gate"]}
        be.graph_compute([ghip.mul_mat_node(ws[nm], ty, kk, src[nm], outs[nm]) for nm, ty, kk, _ in shapes])
        torch.cuda.synchronize()
        return outs, src

    got, src = run()
    monkeypatch.setenv("GHIP_GRAPH_PREQUANT", "0")
    want, _ = run()
    for nm, ty, kk, _ in shapes:
        assert torch.equal(got[nm], want[nm]), nm
        single = be.mul_mat(ws[nm], ty, kk, src[nm])
        torch.cuda.synchronize()
        assert torch.equal(got[nm], single), nm


def test_prequantized_inputs_past_eight(be, monkeypatch):
    """More than 8 independent inputs: the first 8 are quantized up front in
    one launch, the rest by their own nodes; every output equals the result
    without the pre-pass and ghip_mul_mat's (4 activation rows, Q4_K and
    Q6_K nodes, ragged row counts)."""
    import ghip
    k, m = 512, 4
    g = torch.Generator(device="cuda").manual_seed(77)
    specs = [(12 if i % 3 else 14, 64 + 40 * i) for i in range(10)]
    ws = [weights(be, ty, n, k, 100 + i) for i, (ty, n) in enumerate(specs)]
    xs = [torch.randn((m, k), device="cuda", generator=g) for _ in specs]
    print("prequantized inputs past eight", flush=True)

    def run():
        outs = [torch.full((m, n), float("nan"), device="cuda") for _, n in specs]
        be.graph_compute([ghip.mul_mat_node(w, ty, k, x, o) for w, (ty, _), x, o in zip(ws, specs, xs, outs)])
        torch.cuda.synchronize()
        return outs

    got = run()
    monkeypatch.setenv("GHIP_GRAPH_PREQUANT", "0")
    want = run()
    for i, (ty, _) in enumerate(specs):
        assert torch.equal(got[i], want[i]), i
        single = be.mul_mat(ws[i], ty, k, xs[i])
        torch.cuda.synchronize()
        assert torch.equal(got[i], single), i
