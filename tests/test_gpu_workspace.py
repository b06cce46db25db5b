"""Workspace contract (include/ghip.h conventions): growth outside capture
only, outgrown buffers kept for graphs captured earlier, caller-supplied
workspaces, the size query, and ordering across streams."""
import numpy as np
import pytest

import oracle_lib as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture()
def be():
    import ghip
    b = ghip.Backend(0)
    yield b
    b.close()


def weights(be, n, rows, seed):
    import ghip
    g = torch.Generator(device="cuda").manual_seed(seed)
    return be.quantize(torch.randn((rows, n), device="cuda", generator=g) * 0.02, ghip.Q6_K)


def test_graph_survives_growth(be):
    """A graph captured with a small workspace replays correctly after a
    bigger call has grown (and replaced) the workspace."""
    import ghip
    n, rows = 1024, 256
    w = weights(be, n, rows, 1)
    x = torch.randn((2, n), device="cuda")
    out = torch.empty((2, rows), device="cuda")
    # Q6_K at 2 columns: separate Q8_K quantization into the workspace
    be.mul_mat(w, ghip.Q6_K, n, x, out=out)
    torch.cuda.synchronize()
    ref = out.clone()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        be.mul_mat(w, ghip.Q6_K, n, x, out=out)  # warm: no growth inside the capture
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            be.mul_mat(w, ghip.Q6_K, n, x, out=out)
    torch.cuda.synchronize()
    # a much bigger call: the Q6_K GEMM's workspace replaces the small one
    big_w = weights(be, 4096, 512, 2)
    big_x = torch.randn((256, 4096), device="cuda")
    be.mul_mat(big_w, ghip.Q6_K, 4096, big_x)
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        be.mul_mat(big_w, ghip.Q6_K, 4096, big_x)  # eager work between replays
        torch.cuda.synchronize()


def test_growth_during_capture_fails(be):
    import ghip
    n, rows = 4096, 512
    w = weights(be, n, rows, 3)
    x = torch.randn((256, n), device="cuda")
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(ghip.GhipError, match="captured"):
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                be.mul_mat(w, ghip.Q6_K, n, x)
    torch.cuda.synchronize()


def test_caller_workspace(be):
    import ghip
    n, rows, cols = 2048, 384, 96
    w = weights(be, n, rows, 4)
    x = torch.randn((cols, n), device="cuda")
    out = torch.empty((cols, rows), device="cuda")
    node = ghip.mul_mat_node(w, ghip.Q6_K, n, x, out)
    need = be.workspace_size(node)
    assert need > 0
    want = be.mul_mat(w, ghip.Q6_K, n, x).clone()
    buf = torch.empty(need, dtype=torch.uint8, device="cuda")
    be.set_workspace(buf)
    be.mul_mat(w, ghip.Q6_K, n, x, out=out)
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    be.set_workspace(torch.empty(need - 256, dtype=torch.uint8, device="cuda"))
    with pytest.raises(ghip.GhipError, match="set_workspace"):
        be.mul_mat(w, ghip.Q6_K, n, x, out=out)
    be.set_workspace(None)
    be.mul_mat(w, ghip.Q6_K, n, x, out=out)
    torch.cuda.synchronize()
    assert torch.equal(out, want)


def test_caller_workspace_graph(be):
    """A caller's workspace sized by ghip_workspace_size (the largest node)
    covers a ghip_graph_compute call whose whole-K decode groups would
    otherwise have their inputs quantized up front (that keeps Q8_K rows
    ahead of the nodes' workspace, so it is off with a caller's workspace):
    same bits as with the library's own workspace."""
    import ghip
    k, m = 2048, 8
    g = torch.Generator(device="cuda").manual_seed(21)
    shapes = [("q", 1024), ("k", 256), ("o", 1024), ("gate", 3072)]
    ws = {nm: be.quantize(torch.randn((n, k), device="cuda", generator=g) * 0.02, ghip.Q4_K) for nm, n in shapes}
    xs = {"x": torch.randn((m, k), device="cuda", generator=g), "xo": torch.randn((m, k), device="cuda", generator=g),
          "xf": torch.randn((m, k), device="cuda", generator=g)}
    src = {"q": "x", "k": "x", "o": "xo", "gate": "xf"}
    print("caller workspace graph", flush=True)

    def run():
        outs = {nm: torch.full((m, n), float("nan"), device="cuda") for nm, n in shapes}
        nodes = [ghip.mul_mat_node(ws[nm], ghip.Q4_K, k, xs[src[nm]], outs[nm]) for nm, _ in shapes]
        be.graph_compute(nodes)
        torch.cuda.synchronize()
        return outs, nodes

    want, nodes = run()
    need = max(be.workspace_size(nd) for nd in nodes)
    be.set_workspace(torch.empty(max(need, 256), dtype=torch.uint8, device="cuda"))
    got, _ = run()
    be.set_workspace(None)
    for nm, _ in shapes:
        assert torch.equal(got[nm], want[nm]), nm


def test_two_streams(be):
    """Back-to-back calls on two streams share the workspace safely (the second
    stream waits for the first)."""
    import ghip
    n, rows = 4096, 1024
    ws = [weights(be, n, rows, 10 + i) for i in range(2)]
    xs = [torch.randn((3, n), device="cuda") for _ in range(2)]
    want = [be.mul_mat(ws[i], ghip.Q6_K, n, xs[i]).clone() for i in range(2)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [torch.empty((3, rows), device="cuda") for _ in range(2)]
    for it in range(20):
        for i in range(2):
            with torch.cuda.stream(streams[i]):
                be.mul_mat(ws[i], ghip.Q6_K, n, xs[i], out=outs[i])
    torch.cuda.synchronize()
    for i in range(2):
        assert torch.equal(outs[i], want[i])
