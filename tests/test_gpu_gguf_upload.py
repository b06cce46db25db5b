"""GGUF -> device upload (ghip_gguf_upload): a file written with Q6_K, Q4_K
and MXFP4 weights is uploaded, optionally registered (the device-side repack
of the reference's load-time CPU_REPACK), and used by MUL_MAT / MUL_MAT_ID;
results are bit-identical to the same bytes placed on the device by torch,
and the uploaded bytes equal the file's."""
import os

import numpy as np
import pytest

import gguf_py as G
import oracle_lib as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def be():
    import ghip
    b = ghip.Backend(0)
    yield b
    b.close()


def test_upload_register_and_use(be, tmp_path):
    import ghip
    rng = np.random.default_rng(0)
    n, rows = 1024, 96
    w6 = O.quantize(O.Q6_K, (rng.standard_normal((rows, n)) * 0.02).astype(np.float32)).reshape(rows, -1)
    w4 = O.quantize(O.Q4_K, (rng.standard_normal((rows, n)) * 0.02).astype(np.float32)).reshape(rows, -1)
    n_as, er = 4, 64
    wx = be.quantize(torch.from_numpy((rng.standard_normal((n_as * er, n)) * 0.02).astype(np.float32)).cuda(),
                     ghip.MXFP4).cpu().numpy().reshape(n_as, er, -1)
    path = str(tmp_path / "w.gguf")
    G.write(path, [("general.architecture", G.STR, "test")],
            [("ffn_down", 14, [n, rows], w6.tobytes()), ("attn_q", 12, [n, rows], w4.tobytes()),
             ("ffn_gate_exps", 39, [n, er, n_as], wx.tobytes())], alignment=32)
    g = ghip.Gguf(path)
    print(f"gguf upload n={n} rows={rows} experts={n_as}x{er}", flush=True)
    base = be.weight_cache_stats()
    d6 = g.upload(be, "ffn_down", register=True)
    d4 = g.upload(be, "attn_q", register=True)
    dx = g.upload(be, "ffn_gate_exps", register=True)
    assert d6.shape == (rows, w6.shape[1]) and dx.shape == (n_as, er, wx.shape[2])
    assert np.array_equal(d6.cpu().numpy(), w6) and np.array_equal(dx.cpu().numpy(), wx)
    n1, _, built = be.weight_cache_stats()
    assert n1 == base[0] + 2 and built == base[2] + 2  # Q6_K and MXFP4 keep copies; Q4_K needs none
    x = torch.from_numpy(rng.standard_normal((80, n)).astype(np.float32)).cuda()  # GEMM route for Q6_K
    t6 = torch.from_numpy(w6).cuda()
    assert torch.equal(be.mul_mat(d6, O.Q6_K, n, x), be.mul_mat(t6, O.Q6_K, n, x))
    assert torch.equal(be.mul_mat(d4, O.Q4_K, n, x), be.mul_mat(torch.from_numpy(w4).cuda(), O.Q4_K, n, x))
    b = torch.from_numpy(rng.standard_normal((16, 1, n)).astype(np.float32)).cuda()
    ids = torch.from_numpy(np.stack([rng.permutation(n_as)[:2] for _ in range(16)]).astype(np.int32)).cuda()
    assert torch.equal(be.mul_mat_id(dx, n, b, ids), be.mul_mat_id(torch.from_numpy(wx).cuda(), n, b, ids))
    for t, ty in ((d6, O.Q6_K), (dx, ghip.MXFP4)):
        be.unregister_weight(t, ty, n)
    assert be.weight_cache_stats()[:2] == base[:2]
