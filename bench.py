"""bench.py -- llama.rust quantized ggml hot path on one MI355X.

Step (timed): one Llama-3-8B decode layer's MUL_MAT set at batch 1 --
q, k, v, o, gate, up (Q4_K) and down (Q6_K) -- each op including its on-device
Q8_K activation quantization, weights rotated over 4 layer copies (551 MB) so
the 256 MB Infinity Cache cannot serve them.  The step is one
ghip_graph_compute call over the 7 nodes (the reference's graph-level seam,
which runs q/k/v and gate/up as one launch each); the same 7 nodes as
separate ghip_mul_mat calls are reported beside it.
value = algorithmic bytes of the step (weights + f32 activations in + f32
outputs, BASELINE's per-matrix formula) / step time.

Also reported: the same set at batch 2/4/8, and the roofline of the dominant
kernel (the Q4_K 4096->14336 GEMV on pre-quantized activations, HIP events on
the launch stream, 16 rotating weight copies), and the CPU baseline (the C
restatement of llama.rust's CPU path, all host threads).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "llama.rust_amd"))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
METRIC = "Q4_K GEMV GB/s (% of 8 TB/s HBM) + Q4_K prefill GEMM TOPS (% MFMA peak)"

LAYER = [  # (name, weight type, K, N)
    ("q", 12, 4096, 4096), ("k", 12, 4096, 1024), ("v", 12, 4096, 1024), ("o", 12, 4096, 4096),
    ("gate", 12, 4096, 14336), ("up", 12, 4096, 14336), ("down", 14, 14336, 4096),
]
# the activation each node reads, as in the model: q/k/v the attention-norm
# output, o the attention output, gate/up the FFN-norm output, down the
# gated FFN activation (so only q/k/v and gate/up share an input)
LAYER_INPUT = {"q": "x_attn", "k": "x_attn", "v": "x_attn", "o": "attn_out", "gate": "x_ffn", "up": "x_ffn",
               "down": "h_ffn"}
INPUT_K = {"x_attn": 4096, "attn_out": 4096, "x_ffn": 4096, "h_ffn": 14336}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_weights(be, torch, np, copies):
    """GGUF-quantized weights ~N(0, 0.02) from seed 0, quantized on the GPU."""
    import ghip
    rng = np.random.default_rng(0)
    layer = []
    for name, ty, k, n in LAYER:
        wf = torch.from_numpy((rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))).cuda()
        layer.append(be.quantize(wf, ty))
        del wf
    sets = [layer] + [[w.clone() for w in layer] for _ in range(copies - 1)]
    torch.cuda.synchronize()
    return sets


def weight_bytes(ty, k, n):
    import ghip
    return ghip.row_size(ty, k) * n


def step_bytes(batch):
    return sum(weight_bytes(ty, k, n) + batch * k * 4 + batch * n * 4 for _, ty, k, n in LAYER)


def time_layer(be, torch, sets, xs, outs, steps, warmup, graph=False):
    """Seconds per decode-layer step.  Each step is one replay of a HIP graph
    holding the layer's 7 MUL_MATs (quantization + kernel each) for one of
    the weight copies, so host launch gaps are not in the measurement.
    graph=False: one ghip_mul_mat call per node; graph=True: one
    ghip_graph_compute call over the 7 nodes (the reference's graph-level
    seam), which runs q/k/v and gate/up as one launch each."""
    import ghip
    node_lists = [[ghip.mul_mat_node(w, ty, k, xs[LAYER_INPUT[name]], outs[name]) for (name, ty, k, n), w in zip(LAYER, ws)]
                  for ws in sets]

    def one(i):
        if graph:
            be.graph_compute(node_lists[i % len(sets)])
            return
        ws = sets[i % len(sets)]
        for (name, ty, k, n), w in zip(LAYER, ws):
            be.mul_mat(w, ty, k, xs[LAYER_INPUT[name]], out=outs[name])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(len(sets)):
            one(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graphs = []
    for i in range(len(sets)):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            one(i)
        graphs.append(g)
    for i in range(warmup):
        graphs[i % len(graphs)].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        graphs[i % len(graphs)].replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def time_layer_eager(be, torch, sets, xs, outs, steps):
    """Same step issued op by op from Python (host launch cost included)."""
    def one(i):
        ws = sets[i % len(sets)]
        for (name, ty, k, n), w in zip(LAYER, ws):
            be.mul_mat(w, ty, k, xs[LAYER_INPUT[name]], out=outs[name])
    for i in range(3):
        one(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        one(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def graph_time_us(torch, launch, n, reps=5):
    """Average device time of one launch: n launches captured in a HIP graph
    (no host gaps between them), replayed with HIP events on the capture
    stream."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(3):
            launch(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            launch(i)
    g.replay()
    torch.cuda.synchronize()
    best = None
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1000.0 / n
        best = us if best is None else min(best, us)
    return best


def gemv_roofline(be, torch, np, n_launch=64):
    """Average duration of the Q4_K 4096->14336 batch-1 MUL_MAT kernel
    (f32 activations, Q8_K quantization fused), 16 rotating weight copies."""
    import ghip
    k, n = 4096, 14336
    rng = np.random.default_rng(0)
    wf = torch.from_numpy(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).cuda()
    w0 = be.quantize(wf, ghip.Q4_K)
    del wf
    ws = [w0] + [w0.clone() for _ in range(15)]
    x = torch.from_numpy(np.random.default_rng(1).standard_normal((1, k), dtype=np.float32)).cuda()
    out = torch.empty((1, n), dtype=torch.float32, device="cuda")
    us = graph_time_us(torch, lambda i: be.mul_mat(ws[i % 16], ghip.Q4_K, k, x, out=out), n_launch)
    wb = ghip.row_size(ghip.Q4_K, k) * n
    alg = wb + k * 4 + n * 4
    return us, alg, wb


def q4_0_bench(be, torch, np):
    """Config 1 (the reference's CPU-runnable case): Q4_0 4096x4096 batch-1
    MUL_MAT (Q8_0 activation quantization + GEMV), 16 rotating weight copies."""
    import ghip
    k = n = 4096
    rng = np.random.default_rng(0)
    wf = torch.from_numpy(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).cuda()
    w0 = be.quantize(wf, ghip.Q4_0)
    del wf
    ws = [w0] + [w0.clone() for _ in range(31)]  # 32 x 9.4 MB > the 256 MB Infinity Cache
    x = torch.from_numpy(np.random.default_rng(1).standard_normal((1, k), dtype=np.float32)).cuda()
    out = torch.empty((1, n), dtype=torch.float32, device="cuda")
    us = graph_time_us(torch, lambda i: be.mul_mat(ws[i % 32], ghip.Q4_0, k, x, out=out), 64)
    alg = w0.numel() + k * 4 + n * 4
    log(f"Q4_0 4096x4096 GEMV op: {us:.2f} us, {alg / us / 1e3:.1f} GB/s")
    return {"us_op": round(us, 2), "GB/s": round(alg / us / 1e3, 1), "bytes": alg,
            "frac_hbm": round(alg / us / 1e3 / HBM_PEAK_GBS, 4)}


def more_types_bench(be, torch, np):
    """Q5_0 / Q8_0 / Q5_K decode GEMV, 4096 -> 14336 at batch 1 (the gate/up
    shape), 16 rotating weight copies.  Weights are random blocks with finite
    f16 scales built on the device: the kernels' time does not depend on
    the values."""
    import ghip
    k, n = 4096, 14336
    res = {}
    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn((1, k), device="cuda", generator=g)
    out = torch.empty((1, n), dtype=torch.float32, device="cuda")
    for name, ty in (("q5_0", ghip.Q5_0), ("q8_0", ghip.Q8_0), ("q5_K", ghip.Q5_K)):
        qk, bs = ghip.BLOCK[ty]
        w0 = torch.randint(0, 256, (n, k // qk, bs), dtype=torch.uint8, device="cuda", generator=g)
        scale = torch.full((n, k // qk), 0x2000, dtype=torch.int16, device="cuda")  # f16 2^-7
        w0[:, :, 0:2] = scale.view(torch.uint8).view(n, k // qk, 2)
        if ty == ghip.Q5_K:
            w0[:, :, 2:4] = scale.view(torch.uint8).view(n, k // qk, 2)
        w0 = w0.view(n, -1).contiguous()
        copies = max(2, min(16, (512 << 20) // w0.numel()))
        ws = [w0] + [w0.clone() for _ in range(copies - 1)]
        us = graph_time_us(torch, lambda i: be.mul_mat(ws[i % copies], ty, k, x, out=out), 64)
        alg = w0.numel() + k * 4 + n * 4
        log(f"{name} 4096->14336 GEMV op: {us:.2f} us, {alg / us / 1e3:.1f} GB/s")
        res[name] = {"us_op": round(us, 2), "GB/s": round(alg / us / 1e3, 1), "bytes": alg,
                     "frac_hbm": round(alg / us / 1e3 / HBM_PEAK_GBS, 4)}
        del ws, w0
    return res


def measured_traffic():
    """HBM bytes per launch of the dominant kernel: the calibrated
    FETCH_SIZE + WRITE_SIZE that the committed rocprofv3 summary states on its
    `traffic_bytes_per_launch:` line (None when the summary is absent)."""
    path = os.path.join(ROOT, "profiles", "gemv_q4K_4096x14336_b1.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1].strip().replace(",", ""))
    except (OSError, ValueError):
        pass
    return None


def _profile_ops(be, torch, np, what):
    """One launch closure per profiled kernel family, on the bench's shapes."""
    import ghip
    g = torch.Generator(device="cuda").manual_seed(0)
    if what in ("gemv", "gemv_graph", "copy"):
        k, nr = 4096, 14336
        rng = np.random.default_rng(0)
        wf = torch.from_numpy(rng.standard_normal((nr, k), dtype=np.float32) * np.float32(0.02)).cuda()
        w0 = be.quantize(wf, ghip.Q4_K)
        del wf
        ws = [w0] + [w0.clone() for _ in range(15)]
        x = torch.from_numpy(np.random.default_rng(1).standard_normal((1, k), dtype=np.float32)).cuda()
        out = torch.empty((1, nr), dtype=torch.float32, device="cuda")
        if what == "gemv":
            return lambda i: be.mul_mat(ws[i % 16], ghip.Q4_K, k, x, out=out)
        if what == "gemv_graph":
            # the roofline's timing setup: 64 launches in one HIP graph, replayed
            return _graph_replay(torch, lambda i: be.mul_mat(ws[i % 16], ghip.Q4_K, k, x, out=out), 64)
        # one 33,030,144-byte device-to-device copy per launch
        return lambda i: ws[(i + 1) % 16].copy_(ws[i % 16])
    if what in ("gemm", "gemm_q6k", "gemm_q4_0", "decode_b8"):
        ty, m, k, n = {"gemm": (ghip.Q4_K, 512, 4096, 14336), "gemm_q6k": (ghip.Q6_K, 512, 14336, 4096),
                       "gemm_q4_0": (ghip.Q4_0, 512, 4096, 14336), "decode_b8": (ghip.Q4_K, 8, 4096, 14336)}[what]
        copies = 16 if what == "decode_b8" else 1
        wf = torch.randn((n, k), device="cuda", generator=g) * 0.02
        ws = [be.quantize(wf, ty)]
        del wf
        ws += [ws[0].clone() for _ in range(copies - 1)]
        if ty == ghip.Q4_0:  # registered: the GEMM reads the kept int8 codes
            be.register_weight(ws[0], ty, k)
        x = torch.randn((m, k), device="cuda", generator=g)
        out = torch.empty((m, n), dtype=torch.float32, device="cuda")
        return lambda i: be.mul_mat(ws[i % copies], ty, k, x, out=out)
    if what in ("layer_b1", "layer_b8"):
        batch = 1 if what == "layer_b1" else 8
        sets = make_weights(be, torch, np, copies=4)
        xr = np.random.default_rng(1)
        xs = {nm: torch.from_numpy(xr.standard_normal((batch, k), dtype=np.float32)).cuda() for nm, k in INPUT_K.items()}
        outs = {name: torch.empty((batch, n), dtype=torch.float32, device="cuda") for name, _, _, n in LAYER}
        nodes = [[ghip.mul_mat_node(w, ty, k, xs[LAYER_INPUT[name]], outs[name])
                  for (name, ty, k, n), w in zip(LAYER, ws)] for ws in sets]
        return lambda i: be.graph_compute(nodes[i % len(nodes)])
    if what in ("moe", "moe_reg"):
        n_as, n_tok, n_ids, k, rows = 32, 256, 4, 2880, 5760
        rng = np.random.default_rng(3)
        ids = torch.from_numpy(np.argsort(-rng.standard_normal((n_tok, n_as)), axis=1)[:, :n_ids]
                               .astype(np.int32)).cuda()
        wf = torch.randn((n_as * rows, k), device="cuda", generator=g) * 0.02
        w = be.quantize(wf, ghip.MXFP4).view(n_as, rows, -1)
        del wf
        b = torch.randn((n_tok, 1, k), device="cuda", generator=g)
        out = torch.empty((n_tok, n_ids, rows), dtype=torch.float32, device="cuda")
        if what == "moe_reg":  # experts registered: the kernel reads the repacked windows
            be.register_weight(w, ghip.MXFP4, k)
        return lambda i: be.mul_mat_id(w, k, b, ids, out=out)
    if what in ("fa_decode", "fa_prefill"):
        H, Hkv, D, S = 32, 8, 128, 8192
        T = 1 if what == "fa_decode" else 512
        kk = torch.randn((Hkv, S, D), device="cuda", generator=g).half()
        v = torch.randn((Hkv, S, D), device="cuda", generator=g).half()
        q = torch.randn((H, T, D), device="cuda", generator=g)
        mask = torch.zeros((T, S), dtype=torch.float16, device="cuda")
        for t in range(T):
            mask[t, S - T + t + 1:] = float("-inf")
        out = torch.empty((T, H, D), dtype=torch.float32, device="cuda")
        return lambda i: be.flash_attn_ext(q, kk, v, mask, None, 1.0 / D ** 0.5, out=out)
    raise ValueError(what)


def _graph_replay(torch, launch, n):
    """Capture n launches in a HIP graph (after 3 eager warm-up launches) and
    return a closure that replays it; launch i of the profile loop replays
    the whole graph when i % n == 0, so L launches are L // n replays."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(3):
            launch(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            launch(i)
    torch.cuda.synchronize()
    return lambda i: g.replay() if i % n == 0 else None


PROFILE_WORKLOADS = ["gemv", "gemv_graph", "copy", "gemm", "gemm_q6k", "gemm_q4_0", "decode_b8", "layer_b1", "layer_b8", "moe", "moe_reg",
                     "fa_decode", "fa_prefill"]


def profile_loop(what, n):
    """Plain launch loops for rocprofv3 runs (no JSON): one kernel family on
    the bench's shape, or the copy kernel used to calibrate FETCH_SIZE /
    WRITE_SIZE.  gemv: Q4_K 4096->14336 at batch 1 over 16 weight copies;
    gemv_graph: the same launches captured 64 to a HIP graph and replayed
    (the roofline's steady state, no first-touch launches);
    copy: 33,030,144-byte device copies; gemm: Q4_K 512x4096->14336;
    gemm_q6k: Q6_K 512x14336->4096; decode_b8: Q4_K 4096->14336 at 8 rows over
    16 copies; layer_b1 / layer_b8: the decode layer's 7 MUL_MATs in one
    graph_compute call at batch 1 / 8 over 4 weight copies; moe / moe_reg: MXFP4 gate_up (32 experts, 256 tokens, top-4; moe_reg with the experts registered);
    fa_decode / fa_prefill: FLASH_ATTN_EXT 32/8 heads, D 128, KV 8192, T 1 / 512."""
    import numpy as np
    import torch
    import ghip
    be = ghip.Backend(0)
    launch = _profile_ops(be, torch, np, what)
    torch.cuda.synchronize()
    for i in range(n):
        launch(i)
    torch.cuda.synchronize()
    print(f"profile {what}: {n} launches", file=sys.stderr)


def gemm_bench(be, torch, np):
    """Config 3: Q4_K prefill MUL_MAT (Q8_K quantization + int8 MFMA GEMM)."""
    import ghip
    res = {}
    g = torch.Generator(device="cuda").manual_seed(0)
    for m, k, n in [(512, 4096, 14336), (128, 4096, 4096), (2048, 4096, 4096)]:
        wf = torch.randn((n, k), device="cuda", generator=g) * 0.02
        w = be.quantize(wf, ghip.Q4_K)
        del wf
        x = torch.randn((m, k), device="cuda", generator=g)
        out = torch.empty((m, n), dtype=torch.float32, device="cuda")
        act = be.mul_mat_act(w, ghip.Q4_K, k, x)
        us_op = graph_time_us(torch, lambda i: be.mul_mat(w, ghip.Q4_K, k, x, out=out), 10)
        us_k = graph_time_us(torch, lambda i: be.mul_mat(w, ghip.Q4_K, k, act, out=out), 10)
        ops = 2.0 * m * n * k
        res[f"{m}x{k}->{n}"] = {"us_op": round(us_op, 2), "us_gemm_kernel": round(us_k, 2),
                                "TOPS_op": round(ops / us_op / 1e6, 1), "TOPS_gemm_kernel": round(ops / us_k / 1e6, 1),
                                "frac_int8_peak_kernel": round(ops / us_k / 1e6 / INT8_PEAK_TOPS, 4)}
        log(f"GEMM {m}x{k}->{n}: op {us_op:.1f} us ({ops / us_op / 1e6:.1f} TOPS), kernel {us_k:.1f} us "
            f"({ops / us_k / 1e6:.1f} TOPS)")
        del w, x, out, act
    return res


def gemm_q6k_bench(be, torch, np):
    """The Q4_K_M down projection at 512 tokens (Q6_K 14336 -> 4096): the
    f16-MFMA GEMM (weight repack + f16 code layout + GEMM), the same with
    the weight registered (repack kept on the device, as the reference's
    repack cache), and the 8-column decode kernels it replaces."""
    import ghip
    m, k, n = 512, 14336, 4096
    g = torch.Generator(device="cuda").manual_seed(0)
    wf = torch.randn((n, k), device="cuda", generator=g) * 0.02
    w = be.quantize(wf, ghip.Q6_K)
    del wf
    x = torch.randn((m, k), device="cuda", generator=g)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    us = graph_time_us(torch, lambda i: be.mul_mat(w, ghip.Q6_K, k, x, out=out), 10)
    be.register_weight(w, ghip.Q6_K, k)  # the repacked records kept on the device
    us_reg = graph_time_us(torch, lambda i: be.mul_mat(w, ghip.Q6_K, k, x, out=out), 10)
    be.unregister_weight(w, ghip.Q6_K, k)
    os.environ["GHIP_GEMM_Q6K_MIN_ROWS"] = str(1 << 30)
    try:
        us_gemv = graph_time_us(torch, lambda i: be.mul_mat(w, ghip.Q6_K, k, x, out=out), 2, reps=2)
    finally:
        del os.environ["GHIP_GEMM_Q6K_MIN_ROWS"]
    ops = 2.0 * m * n * k
    log(f"Q6_K GEMM {m}x{k}->{n}: op {us:.1f} us ({ops / us / 1e6:.1f} TOPS), registered weight {us_reg:.1f} us "
        f"({ops / us_reg / 1e6:.1f} TOPS); 8-column decode kernels {us_gemv:.1f} us")
    return {f"{m}x{k}->{n}": {"us_op": round(us, 2), "TOPS_op": round(ops / us / 1e6, 1),
                              "frac_f16_peak": round(ops / us / 1e6 / 2500.0, 4),
                              "us_op_registered_weight": round(us_reg, 2),
                              "TOPS_op_registered_weight": round(ops / us_reg / 1e6, 1),
                              "us_op_8col_decode_kernels": round(us_gemv, 2)}}


def gemm_q8_family_bench(be, torch, np):
    """Prefill of 32-element-block weights (Q4_0, Q8_0) and Q5_K at 512
    tokens, 4096 -> 14336: the int8-MFMA GEMMs (per-call repack and registered
    weight for the 32-element blocks), against the 8-column decode kernels
    they replace."""
    import ghip
    res = {}
    m, k, n = 512, 4096, 14336
    g = torch.Generator(device="cuda").manual_seed(4)
    for name, ty in (("q4_0", ghip.Q4_0), ("q8_0", ghip.Q8_0)):
        if ty == ghip.Q4_0:
            w = be.quantize(torch.randn((n, k), device="cuda", generator=g) * 0.02, ty)
        else:  # no device Q8_0 quantizer: valid blocks of random codes with a fixed f16 scale
            blk = torch.randint(-127, 128, (n, k // 32, 34), device="cuda", generator=g, dtype=torch.int32)
            blk = blk.to(torch.int8).view(torch.uint8)
            blk[:, :, 0:2] = torch.tensor([0x1A, 0x14], dtype=torch.uint8, device="cuda")  # f16 0.001
            w = blk.reshape(n, -1).contiguous()
        x = torch.randn((m, k), device="cuda", generator=g)
        out = torch.empty((m, n), dtype=torch.float32, device="cuda")
        us = graph_time_us(torch, lambda i: be.mul_mat(w, ty, k, x, out=out), 10)
        be.register_weight(w, ty, k)
        us_reg = graph_time_us(torch, lambda i: be.mul_mat(w, ty, k, x, out=out), 10)
        be.unregister_weight(w, ty, k)
        os.environ["GHIP_GEMM_Q8_MIN_ROWS"] = str(1 << 30)
        try:
            us_gemv = graph_time_us(torch, lambda i: be.mul_mat(w, ty, k, x, out=out), 2, reps=2)
        finally:
            del os.environ["GHIP_GEMM_Q8_MIN_ROWS"]
        ops = 2.0 * m * n * k
        res[f"{name} {m}x{k}->{n}"] = {"us_op": round(us, 2), "us_op_registered_weight": round(us_reg, 2),
                                       "TOPS_op_registered_weight": round(ops / us_reg / 1e6, 1),
                                       "frac_int8_peak": round(ops / us_reg / 1e6 / INT8_PEAK_TOPS, 4),
                                       "us_op_8col_decode_kernels": round(us_gemv, 2)}
        log(f"{name} GEMM {m}x{k}->{n}: op {us:.1f} us, registered {us_reg:.1f} us "
            f"({ops / us_reg / 1e6:.1f} TOPS); 8-column decode kernels {us_gemv:.1f} us")
        del w, x, out
    # Q5_K: the wide Q4_K tiles with the fifth-bit plane (no device Q5_K
    # quantizer: random blocks with small finite d / dmin)
    blk = torch.randint(0, 256, (n, k // 256, 176), device="cuda", generator=g, dtype=torch.int32).to(torch.uint8)
    blk[:, :, 0:4] = torch.tensor([0x1A, 0x14, 0x1A, 0x14], dtype=torch.uint8, device="cuda")  # d, dmin = 0.001
    w = blk.reshape(n, -1).contiguous()
    x = torch.randn((m, k), device="cuda", generator=g)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    us = graph_time_us(torch, lambda i: be.mul_mat(w, ghip.Q5_K, k, x, out=out), 10)
    os.environ["GHIP_GEMM_Q5K_MIN_ROWS"] = str(1 << 30)
    try:
        us_gemv = graph_time_us(torch, lambda i: be.mul_mat(w, ghip.Q5_K, k, x, out=out), 2, reps=2)
    finally:
        del os.environ["GHIP_GEMM_Q5K_MIN_ROWS"]
    ops = 2.0 * m * n * k
    res[f"q5_K {m}x{k}->{n}"] = {"us_op": round(us, 2), "TOPS_op": round(ops / us / 1e6, 1),
                                 "frac_int8_peak": round(ops / us / 1e6 / INT8_PEAK_TOPS, 4),
                                 "us_op_8col_decode_kernels": round(us_gemv, 2)}
    log(f"q5_K GEMM {m}x{k}->{n}: op {us:.1f} us ({ops / us / 1e6:.1f} TOPS); 8-column decode kernels {us_gemv:.1f} us")
    return res


def prefill_layer_bench(be, torch, np, tokens=512):
    """The decode layer's 7 MUL_MAT nodes at `tokens` activation rows (a
    prefill step): q/k/v/o/gate/up on the Q4_K int8 GEMM, down on the Q6_K
    f16 GEMM, one ghip_graph_compute call, each node reading its own input;
    the weights registered as a loaded model's are."""
    import ghip
    g = torch.Generator(device="cuda").manual_seed(7)
    ws = {}
    for name, ty, k, n in LAYER:
        wf = torch.randn((n, k), device="cuda", generator=g) * 0.02
        ws[name] = be.quantize(wf, ty)
        del wf
    xs = {nm: torch.randn((tokens, k), device="cuda", generator=g) for nm, k in INPUT_K.items()}
    outs = {name: torch.empty((tokens, n), dtype=torch.float32, device="cuda") for name, _, _, n in LAYER}
    for name, ty, k, n in LAYER:  # as a loaded model: weights registered (Q6_K keeps its GEMM records)
        be.register_weight(ws[name], ty, k)
    nodes = [ghip.mul_mat_node(ws[name], ty, k, xs[LAYER_INPUT[name]], outs[name]) for name, ty, k, n in LAYER]
    us = graph_time_us(torch, lambda i: be.graph_compute(nodes), 5)
    for name, ty, k, n in LAYER:
        be.unregister_weight(ws[name], ty, k)
    ops = sum(2.0 * tokens * k * n for _, _, k, n in LAYER)
    log(f"prefill layer ({tokens} tokens, 7 MUL_MATs): {us:.1f} us, {ops / us / 1e6:.1f} TOPS")
    del ws, xs, outs, nodes
    return {"tokens": tokens, "us": round(us, 1), "TOPS": round(ops / us / 1e6, 1), "tokens_per_s": round(tokens / us * 1e6, 1)}


def q4_0_layer_bench(be, torch, np, copies=4):
    """The decode layer's 7 MUL_MAT nodes with Q4_0 weights (the Q8_0
    activation path, config 1's type) at batch 1: one ghip_graph_compute call
    against 7 ghip_mul_mat calls, both captured in HIP graphs."""
    import ghip
    g = torch.Generator(device="cuda").manual_seed(9)
    sets = [[be.quantize(torch.randn((n, k), device="cuda", generator=g) * 0.02, ghip.Q4_0) for _, _, k, n in LAYER]
            for _ in range(copies)]
    xs = {nm: torch.randn((1, k), device="cuda", generator=g) for nm, k in INPUT_K.items()}
    outs = {name: torch.empty((1, n), dtype=torch.float32, device="cuda") for name, _, _, n in LAYER}
    nodes = [[ghip.mul_mat_node(w, ghip.Q4_0, k, xs[LAYER_INPUT[name]], outs[name])
              for (name, _, k, n), w in zip(LAYER, ws)] for ws in sets]

    def per_op(i):
        for (name, _, k, n), w in zip(LAYER, sets[i % copies]):
            be.mul_mat(w, ghip.Q4_0, k, xs[LAYER_INPUT[name]], out=outs[name])
    us_g = graph_time_us(torch, lambda i: be.graph_compute(nodes[i % copies]), 8)
    us_op = graph_time_us(torch, per_op, 8)
    wbytes = sum(ghip.row_size(ghip.Q4_0, k) * n + 4 * (k + n) for _, _, k, n in LAYER)
    log(f"Q4_0 decode layer: graph_compute {us_g:.1f} us ({wbytes / us_g / 1e3:.0f} GB/s), per-op calls {us_op:.1f} us")
    del sets, xs, outs, nodes
    return {"us_graph_compute": round(us_g, 1), "GB/s": round(wbytes / us_g / 1e3, 1), "us_per_op_calls": round(us_op, 1)}


def moe_bench(be, torch, np):
    """Config 4: gpt-oss MoE MUL_MAT_ID, 32 MXFP4 experts, 256 tokens, top-4;
    headline with the experts registered (as the reference repacks them at
    load), plus the GGUF-layout time."""
    import ghip
    res = {}
    n_as, n_tok, n_ids, k = 32, 256, 4, 2880
    rng = np.random.default_rng(3)
    ids = torch.from_numpy(np.argsort(-rng.standard_normal((n_tok, n_as)), axis=1)[:, :n_ids].astype(np.int32)).cuda()
    g = torch.Generator(device="cuda").manual_seed(1)
    for name, rows, ne11 in [("gate_up", 5760, 1), ("down", 2880, 4)]:
        wf = torch.randn((n_as * rows, k), device="cuda", generator=g) * 0.02
        w = be.quantize(wf, ghip.MXFP4).view(n_as, rows, -1)
        del wf
        b = torch.randn((n_tok, ne11, k), device="cuda", generator=g)
        out = torch.empty((n_tok, n_ids, rows), dtype=torch.float32, device="cuda")
        us_gguf = graph_time_us(torch, lambda i: be.mul_mat_id(w, k, b, ids, out=out), 10)
        be.register_weight(w, ghip.MXFP4, k)  # the experts kept in the kernel's staging layout
        us = graph_time_us(torch, lambda i: be.mul_mat_id(w, k, b, ids, out=out), 10)
        be.unregister_weight(w, ghip.MXFP4, k)
        wbytes = w.numel()
        flops = 2.0 * n_tok * n_ids * rows * k
        res[name] = {"us": round(us, 2), "us_unregistered_weights": round(us_gguf, 2),
                     "weight_GB/s": round(wbytes / us / 1e3, 1),
                     "TFLOP/s": round(flops / us / 1e6, 1), "tokens_per_s": round(n_tok / us * 1e6, 1),
                     "frac_hbm": round(wbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
        log(f"MoE {name}: {us:.1f} us registered ({us_gguf:.1f} us GGUF layout), weights {wbytes / us / 1e3:.0f} GB/s, "
            f"{flops / us / 1e6:.1f} TFLOP/s")
        del w, b, out
    return res


def fa_bench(be, torch, np):
    """Config 5: FLASH_ATTN_EXT, 32 q / 8 KV heads, D 128, KV 8192, causal."""
    res = {}
    H, Hkv, D, S = 32, 8, 128, 8192
    g = torch.Generator(device="cuda").manual_seed(2)
    k = torch.randn((Hkv, S, D), device="cuda", generator=g).half()
    v = torch.randn((Hkv, S, D), device="cuda", generator=g).half()
    for T in (1, 512):
        q = torch.randn((H, T, D), device="cuda", generator=g)
        mask = torch.zeros((T, S), dtype=torch.float16, device="cuda")
        for t in range(T):
            mask[t, S - T + t + 1:] = float("-inf")
        out = torch.empty((T, H, D), dtype=torch.float32, device="cuda")
        us = graph_time_us(torch, lambda i: be.flash_attn_ext(q, k, v, mask, None, 1.0 / D ** 0.5, out=out), 10)
        kv_bytes = 2 * Hkv * S * D * 2
        keys = sum(S - T + t + 1 for t in range(T))
        flops = 4.0 * keys * D * H
        res[f"T{T}"] = {"us": round(us, 2), "kv_GB/s": round(kv_bytes / us / 1e3, 1),
                        "TFLOP/s": round(flops / us / 1e6, 2), "tokens_per_s": round(T / us * 1e6, 1)}
        log(f"FA T={T}: {us:.1f} us, KV {kv_bytes / us / 1e3:.0f} GB/s, {flops / us / 1e6:.1f} TFLOP/s")
    return res


def cpu_baseline(budget_s=12.0):
    """llama.rust's CPU path for the same Q4_K 4096->14336 batch-1 MUL_MAT (the
    repack gemv route), as the C restatement, OpenMP over the host threads."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    k, n = 4096, 14336
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or os.cpu_count()
    rng = np.random.default_rng(0)
    wf = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
    w = O.quantize(O.Q4_K, wf)
    x = np.random.default_rng(1).standard_normal((1, k), dtype=np.float32)
    O.mul_mat(O.Q4_K, w, k, n, x, 1, nthreads=threads)  # warm-up
    reps, t0 = 0, time.perf_counter()
    while True:
        O.mul_mat(O.Q4_K, w, k, n, x, 1, nthreads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el > budget_s:
            break
    wb = O.row_size(O.Q4_K, k) * n
    alg = wb + k * 4 + n * 4
    return {"value": round(alg * reps / el / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"Q4_K 4096->14336 batch-1 MUL_MAT (repack gemv route incl. Q8_K quantization), "
                      f"{reps} calls in {el:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip the prefill GEMM / MoE / FA lines")
    ap.add_argument("--profile", choices=PROFILE_WORKLOADS, help="launch loop for rocprofv3 (no JSON line)")
    ap.add_argument("--launches", type=int, default=100)
    args = ap.parse_args()
    if args.profile:
        profile_loop(args.profile, args.launches)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the path would shard by weight rows / experts / KV heads (not built)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import ghip

    be = ghip.Backend(0)
    log("building weights ...")
    sets = make_weights(be, torch, np, copies=4)
    xrng = np.random.default_rng(1)
    res_by_batch = {}
    ms_headline = None
    for batch in (1, 2, 4, 8):
        xs = {nm: torch.from_numpy(xrng.standard_normal((batch, k), dtype=np.float32)).cuda()
              for nm, k in INPUT_K.items()}
        outs = {name: torch.empty((batch, n), dtype=torch.float32, device="cuda") for name, _, _, n in LAYER}
        steps = args.steps if batch == 1 else max(10, args.steps // 4)
        t_op = time_layer(be, torch, sets, xs, outs, steps, args.warmup)
        t_graph = time_layer(be, torch, sets, xs, outs, steps, args.warmup, graph=True)
        te = time_layer_eager(be, torch, sets, xs, outs, max(10, steps // 4))
        t = t_graph
        gbs = step_bytes(batch) / t / 1e9
        res_by_batch[batch] = {"ms_per_layer": round(t * 1e3, 4), "GB/s": round(gbs, 1),
                               "tokens_per_s_layer": round(batch / t, 1),
                               "ms_per_layer_per_op_calls": round(t_op * 1e3, 4),
                               "GB/s_per_op_calls": round(step_bytes(batch) / t_op / 1e9, 1),
                               "ms_per_layer_eager_launch": round(te * 1e3, 4)}
        log(f"batch {batch}: graph_compute {t*1e6:.1f} us/layer  {gbs:.1f} GB/s; "
            f"per-op calls {t_op*1e6:.1f} us/layer")
        if batch == 1:
            ms_headline, value = t * 1e3, gbs

    us, alg, wb = gemv_roofline(be, torch, np)
    ach = alg / (us * 1e-6) / 1e9
    log(f"Q4_K 4096x14336 GEMV kernel: {us:.2f} us, {ach:.1f} GB/s ({ach / HBM_PEAK_GBS * 100:.1f}% of HBM)")
    roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
            "kernel": "ghip_gemv_q4_K_f_c1_r1x7s3 (Q4_K 4096->14336, batch 1, f32 activations, Q8_K quantization fused)",
            "avg_us": round(us, 3), "bytes_per_launch": alg}
    extras = {}
    if not args.no_extras:
        del sets
        torch.cuda.empty_cache()
        extras["q4_0_gemv_4096"] = q4_0_bench(be, torch, np)
        extras["gemv_q5_0_q8_0_q5_K"] = more_types_bench(be, torch, np)
        extras["prefill_gemm_q4K"] = gemm_bench(be, torch, np)
        extras["prefill_gemm_q6K"] = gemm_q6k_bench(be, torch, np)
        extras["prefill_gemm_q4_0_q8_0"] = gemm_q8_family_bench(be, torch, np)
        extras["prefill_layer_mul_mats"] = prefill_layer_bench(be, torch, np)
        extras["decode_layer_q4_0"] = q4_0_layer_bench(be, torch, np)
        extras["moe_mxfp4"] = moe_bench(be, torch, np)
        extras["flash_attn_f16kv"] = fa_bench(be, torch, np)
    cpu = None if args.no_cpu else cpu_baseline()
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_headline, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (numpy PCG64: weights N(0,0.02) seed 0 quantized on device, activations N(0,1) seed 1)",
        "config": {"workload": "Llama-3-8B decode layer MUL_MAT set (q,k,v,o,gate,up Q4_K; down Q6_K), batch 1, "
                               "one ghip_graph_compute call per step",
                   "bytes_per_step": step_bytes(1), "weight_copies": 4},
        "roofline": roof, "cpu_baseline": cpu,
        "decode_by_batch": res_by_batch, **extras,
    }
    print(json.dumps(line), flush=True)
    be.close()


if __name__ == "__main__":
    main()
