"""bench.py -- llama.rust quantized ggml hot path on one MI355X.

Step (timed): one Llama-3-8B decode layer's MUL_MAT set at batch 1 --
q, k, v, o, gate, up (Q4_K) and down (Q6_K) -- each op including its on-device
Q8_K activation quantization, weights rotated over 4 layer copies (551 MB) so
the 256 MB Infinity Cache cannot serve them.
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
METRIC = "Q4_K GEMV GB/s (% of 8 TB/s HBM) + Q4_K prefill GEMM TOPS (% MFMA peak)"

LAYER = [  # (name, weight type, K, N)
    ("q", 12, 4096, 4096), ("k", 12, 4096, 1024), ("v", 12, 4096, 1024), ("o", 12, 4096, 4096),
    ("gate", 12, 4096, 14336), ("up", 12, 4096, 14336), ("down", 14, 14336, 4096),
]


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


def time_layer(be, torch, sets, xs, outs, steps, warmup):
    def one(i):
        ws = sets[i % len(sets)]
        for (name, ty, k, n), w in zip(LAYER, ws):
            be.mul_mat(w, ty, k, xs[k], out=outs[name])
    for i in range(warmup):
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
        if el > budget_s or reps >= 5000:
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
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the path shards by weight rows / experts / KV heads, see DESIGN.md", file=sys.stderr)
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
        xs = {k: torch.from_numpy(xrng.standard_normal((batch, k), dtype=np.float32)).cuda() for k in (4096, 14336)}
        outs = {name: torch.empty((batch, n), dtype=torch.float32, device="cuda") for name, _, _, n in LAYER}
        steps = args.steps if batch == 1 else max(10, args.steps // 4)
        t = time_layer(be, torch, sets, xs, outs, steps, args.warmup)
        gbs = step_bytes(batch) / t / 1e9
        res_by_batch[batch] = {"ms_per_layer": round(t * 1e3, 4), "GB/s": round(gbs, 1),
                               "tokens_per_s_layer": round(batch / t, 1)}
        log(f"batch {batch}: {t*1e6:.1f} us/layer  {gbs:.1f} GB/s")
        if batch == 1:
            ms_headline, value = t * 1e3, gbs

    us, alg, wb = gemv_roofline(be, torch, np)
    ach = alg / (us * 1e-6) / 1e9
    log(f"Q4_K 4096x14336 GEMV kernel: {us:.2f} us, {ach:.1f} GB/s ({ach / HBM_PEAK_GBS * 100:.1f}% of HBM)")
    roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "ghip_gemv_q4_K_f_c1 (Q4_K 4096->14336, batch 1, f32 activations, Q8_K quantization fused)",
            "avg_us": round(us, 3), "bytes_per_launch": alg}
    cpu = None if args.no_cpu else cpu_baseline()
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_headline, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (numpy PCG64: weights N(0,0.02) seed 0 quantized on device, activations N(0,1) seed 1)",
        "config": {"workload": "Llama-3-8B decode layer MUL_MAT set (q,k,v,o,gate,up Q4_K; down Q6_K), batch 1",
                   "bytes_per_step": step_bytes(1), "weight_copies": 4},
        "roofline": roof, "cpu_baseline": cpu,
        "decode_by_batch": res_by_batch,
    }
    print(json.dumps(line), flush=True)
    be.close()


if __name__ == "__main__":
    main()
