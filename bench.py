"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline (BASELINE.json metric "Q4 decode GEMV achieved HBM GB/s (% peak)"),
on configs[1]: the Llama-3-8B fused gate/up projection, K=4096 x N=28672,
Q4_K weights, one decode token (M=1), bf16 activations.  A step is one pass
of the path over one token batch: activation quantization + fused GEMV.

`value` is algorithmic bytes (Q4_K weight 144 B / 256 elements + activations
+ output) per second over the timed steps, inputs resident in HBM.  The weight
rotates over enough copies (> 512 MB) that the 256 MB Infinity Cache cannot
hold them, so the figure is HBM bandwidth, not MALL bandwidth.  Launches are
captured in a HIP graph so back-to-back decode GEMVs are timed without host
launch gaps.

Also reported: the roofline of the GEMV kernel alone (HIP events on the
launch stream), the CPU baseline (the Candle-method C restatement in
oracle/, multi-threaded on the host), and a sweep of the other decode shapes.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--sweep] [--cpu-seconds S]
"""
import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "Q4 decode GEMV achieved HBM GB/s (% peak); W4A16 prefill TFLOP/s (% MFMA)"
Q_BYTES = {2: 18 / 32, 8: 34 / 32, 12: 144 / 256}
Q_NAME = {2: "q4_0", 8: "q8_0", 12: "q4_k"}


def gemv_bytes(qt, M, K, N, act_bytes=2):
    """Algorithmic HBM bytes of one GEMV: packed weight once, activations,
    f32 output."""
    return int(N * K * Q_BYTES[qt]) + M * K * act_bytes + M * N * 4


def make_weights(qt, N, K, copies, dev, seed=0x5EED):
    """`copies` distinct SoA weights generated on the GPU (random codes and
    bytes, fp16 scales ~ U(0.001, 0.02))."""
    from ubridge_amd import ops
    g = torch.Generator(device=dev).manual_seed(seed)
    bk = ops.BLOCK[qt]
    nb = N * K // bk
    out = []
    for _ in range(copies):
        w = torch.randint(0, 256, (ops.quant_bytes(qt, N * K),), dtype=torch.uint8, device=dev,
                          generator=g)
        hb = 16 if qt == 12 else 2
        hdr = w[: nb * hb].view(nb, hb)
        d = (torch.rand(nb, generator=g, device=dev) * 0.019 + 0.001).half().view(torch.uint8)
        hdr[:, 0:2] = d.view(nb, 2)
        if qt == 12:
            dm = (torch.rand(nb, generator=g, device=dev) * 0.019 + 0.001).half().view(torch.uint8)
            hdr[:, 2:4] = dm.view(nb, 2)
        if qt == 8:  # int8 codes uniform in -127..127
            q = w[nb * hb:].view(torch.int8)
            q[q == -128] = -127
        out.append(w)
    return out


def time_graph(fn_list, reps, stream):
    """Capture fn_list (one launch sequence per element) into a HIP graph and
    time `reps` replays with events on the launch stream.  Returns seconds
    per element."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for fn in fn_list:
            fn()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / 1e3 / (reps * len(fn_list))


def bench_gemv(qt, M, K, N, dev, copies=None, reps=20, x_dtype=torch.bfloat16):
    """Time the fused GEMV kernel alone (prequantized activations) over
    rotating weight copies.  Returns (seconds per GEMV, algorithmic bytes)."""
    from ubridge_amd import ops
    wbytes = ops.quant_bytes(qt, N * K)
    if copies is None:
        copies = max(3, -(-600_000_000 // wbytes))
    ws = make_weights(qt, N, K, copies, dev)
    x = torch.randn(M, K, device=dev, dtype=x_dtype)
    mms = [ops.QMatMul(qt, w, N, K) for w in ws]
    ws0 = mms[0].workspace(M)
    for mm in mms:
        mm._ws = ws0
    mms[0].quantize(x)
    y = torch.empty(M, N, device=dev, dtype=torch.float32)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for mm in mms:  # warm up / validate
            mm.matmul_prequantized(M, y, stream=s)
    torch.cuda.synchronize()
    t = time_graph([lambda mm=mm: mm.matmul_prequantized(M, y, stream=s) for mm in mms], reps, s)
    del ws
    return t, gemv_bytes(qt, M, K, N, 2 if x_dtype == torch.bfloat16 else 4)


def cpu_baseline(qt, K, N, seconds, nthreads):
    """Candle-method QMatMul (oracle/ C restatement) on the host cores, one
    token through the full [N, K] weight, repeated for ~`seconds`."""
    import oracle
    from ubridge_amd import synth
    w = synth.make_weight_soa(qt, N, K, seed=1)
    x = synth.make_activations(1, K, seed=2)
    oracle.qmatmul(qt, w, x, N, K, nthreads)  # warm caches / threads
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.qmatmul(qt, w, x, N, K, nthreads)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per = el / n
    return {"value": round(gemv_bytes(qt, 1, K, N, 4) / per / 1e9, 3), "unit": "GB/s",
            "cores": nthreads, "kind": "port",
            "sample": f"{n} x one-token Candle-method QMatMul ({Q_NAME[qt]}, K={K}, N={N}, "
                      f"f32 act -> Q8_K) in {el:.1f} s, {per * 1e3:.2f} ms each"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--sweep", action="store_true", help="also time every decode shape")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus} requested); the path is "
              "single-GPU by design in this build", file=sys.stderr)
        sys.exit(2)

    import ubridge_amd
    from ubridge_amd import ops
    dev = torch.device("cuda:0")
    qt, M, K, N = ops.Q4_K, 1, 4096, 28672

    # ---- timed steps: quantize activations + fused GEMV, rotating weights
    wbytes = ops.quant_bytes(qt, N * K)
    copies = max(3, -(-600_000_000 // wbytes))
    ws = make_weights(qt, N, K, copies, dev)
    mms = [ops.QMatMul(qt, w, N, K) for w in ws]
    shared_ws = mms[0].workspace(M)
    for mm in mms:
        mm._ws = shared_ws
    x = torch.randn(M, K, device=dev, dtype=torch.bfloat16)
    y = torch.empty(M, N, device=dev, dtype=torch.float32)
    s = torch.cuda.Stream()

    def step(i):
        mms[i % copies].forward(x, out=y, stream=s)

    with torch.cuda.stream(s):
        for i in range(args.warmup):
            step(i)
    torch.cuda.synchronize()
    # one graph holding `copies` steps, replayed to cover args.steps steps
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(copies):
            step(i)
    reps = max(1, args.steps // copies)
    steps = reps * copies
    g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g_e0 = torch.cuda.Event(enable_timing=True)
    g_e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):  # replay() launches on the current stream
        g_e0.record(s)
        for _ in range(reps):
            g.replay()
        g_e1.record(s)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    elapsed = g_e0.elapsed_time(g_e1) / 1e3
    per_step = elapsed / steps
    algo = gemv_bytes(qt, M, K, N)
    value = algo / per_step / 1e9

    # ---- roofline of the dominant kernel: GEMV alone (events on its stream)
    t_k, kbytes = bench_gemv(qt, M, K, N, dev, copies=copies, reps=max(2, reps))
    achieved = kbytes / t_k / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": "k_gemv_q4_k<1,4,f32>", "avg_us": round(t_k * 1e6, 3),
                "bytes_per_launch": kbytes}

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": steps, "warmup": args.warmup, "ms_per_step": round(per_step * 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded random Q4_K blocks, N(0,1) bf16 activations)",
        "config": {"workload": "decode_gemv q4_k K=4096 N=28672 (Llama-3-8B fused gate/up)",
                   "M": M, "K": K, "N": N, "weight_format": "GGUF Q4_K, reference SoA layout",
                   "act_dtype": "bf16", "weight_copies_rotated": copies,
                   "hbm_percent_of_peak": round(100 * value / HBM_PEAK_GBS, 2),
                   "timed_wall_s": round(wall, 4)},
        "roofline": roofline,
    }
    if args.sweep:
        sweep = {}
        for sqt in (ops.Q8_0, ops.Q4_K):
            for (sk, sn) in ((4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)):
                for sm in (1, 4, 16):
                    t, b = bench_gemv(sqt, sm, sk, sn, dev, reps=5)
                    sweep[f"{Q_NAME[sqt]}_K{sk}_N{sn}_M{sm}"] = {
                        "us": round(t * 1e6, 2), "GB/s": round(b / t / 1e9, 1)}
        t, b = bench_gemv(ops.Q4_0, 1, 4096, 4096, dev, reps=5, x_dtype=torch.float32)
        sweep["q4_0_K4096_N4096_M1_f32act(cfg0)"] = {"us": round(t * 1e6, 2),
                                                      "GB/s": round(b / t / 1e9, 1)}
        line["sweep"] = sweep
    if not args.no_cpu:
        nthreads = min(16, os.cpu_count() or 1)
        line["cpu_baseline"] = cpu_baseline(qt, K, N, args.cpu_seconds, nthreads)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
