"""GPU weight quantizers (ghip_quantize_chunk) byte-identical to the CPU ones.

The CPU quantizers are pinned on parity/quants_ref.bin and quants_ref_fp4.bin
(test_oracle_golden.py); the same fixture input is replayed here on the GPU.
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


@pytest.mark.parametrize("ty", [O.Q4_0, O.Q4_K, O.Q6_K, O.MXFP4])
def test_fixture_input(be, ty):
    x = fx.ref_input(1024)
    got = be.quantize(torch.from_numpy(x).cuda().view(1, -1), ty).cpu().numpy().reshape(-1)
    secs = {tid: q for (m, tid, n, q, d) in fx.quant_sections(
        "quants_ref_fp4.bin" if ty == O.MXFP4 else "quants_ref.bin") if n == 1024 and m == 0x54434553}
    assert np.array_equal(got, secs[ty])


@pytest.mark.parametrize("ty", [O.Q4_0, O.Q4_K, O.Q6_K, O.MXFP4])
def test_random_and_edge_blocks(be, ty):
    rng = np.random.default_rng(11)
    rows, n = 96, 2048
    x = (rng.standard_normal((rows, n)) * 0.02).astype(np.float32)
    x[0, :256] = 0.0                     # all-zero blocks
    x[1, :256] = 0.125                   # constant block
    x[2, :] *= 1000.0                    # large magnitudes
    x[3, 5] = 7.0                        # one outlier
    x[4, :] = rng.standard_normal(n).astype(np.float32) * 1e-30  # tiny values
    print(f"quantize type={ty} rows={rows} n={n}", flush=True)
    got = be.quantize(torch.from_numpy(x).cuda(), ty).cpu().numpy().reshape(-1)
    want = O.quantize(ty, x)
    bs = O.BLOCK[ty][1]
    bad = np.nonzero((got != want).reshape(-1, bs).any(1))[0]
    per_row = n // O.BLOCK[ty][0]
    detail = [(int(b // per_row), int(b % per_row), got.reshape(-1, bs)[b][:20].tolist(),
               want.reshape(-1, bs)[b][:20].tolist()) for b in bad[:3]]
    assert bad.size == 0, f"{bad.size} blocks differ (row, block, got, want): {detail}"
