"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline (BASELINE.json metric, first half: "Q4 decode GEMV achieved HBM
GB/s (% peak)"), on configs[1]: the Llama-3-8B fused gate/up projection,
K=4096 x N=28672, Q4_K weights in the reference SoA layout, one decode token
(M=1), bf16 activations.  A step is one pass of the path over one token:
activation quantization (Q8_K) + fused dequant-GEMV, which ubridge_qmatmul
runs as one kernel for Q4_K at M <= 4, K <= 4096 (each workgroup quantizes the
activation chunk it needs while its weight loads are in flight).

`value` = algorithmic bytes per step (Q4_K weight at 144 B / 256 elements +
bf16 activations + f32 output) / measured time per step, inputs resident in
HBM.  The weight rotates over > 512 MB of distinct copies so the 256 MB
Infinity Cache cannot serve it: the figure is HBM bandwidth.  Exactly
--steps steps are captured in one HIP graph and replayed once inside the
timed region, so decode-sized launches are timed back to back without host
gaps.

Also in the line:
  roofline      the step's kernel: median per step over 60 individually
                event-timed replays of a 60-step graph (HIP events on its
                launch stream; the replays hold only back-to-back launches
                of it)
  gemv_prequantized  the GEMV kernel alone, activations quantized beforehand
  cpu_baseline  the Candle-method QMatMul restated in C (oracle/), threaded
                over this process's CPU share, one bf16-valued token through
                the same weight; `secondary` the oracle's GEMMs of
                configs[2]-[4] on bounded row / token samples
  secondary     the other configs: 16-token decode at the headline shape,
                W4A16 prefill TFLOP/s (second half of
                the metric, configs[2] at 512 / 2048 tokens, and 64; GPTQ
                layout and the reference's matmul_bf16_4bit layout, which
                also reports its one-token decode GEMV; each entry names its
                route, and beyond 1024 tokens the pipelined kernel alone is
                reported beside the default slab + hipBLASLt route), fp8
                W8A8 TFLOP/s, W8A16 fused MoE,
                Q4_0 4096x4096 and at 16 tokens on
                4096x28672, QMatMul at 512 and 64 tokens
                (the pipelined GEMM with the Q4_K producer), and
                decode_sweep_cfg1: every decode shape of configs[1] (Q8_0
                and Q4_K, M = 1, 4, 16) with its fraction of HBM peak

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-secondary]
"""
import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0
METRIC = "Q4 decode GEMV achieved HBM GB/s (% peak); W4A16 prefill TFLOP/s (% MFMA)"
Q_BYTES = {2: 18 / 32, 8: 34 / 32, 12: 144 / 256}
Q_NAME = {2: "q4_0", 8: "q8_0", 12: "q4_k"}


def gemv_bytes(qt, M, K, N, act_bytes=2):
    """Algorithmic HBM bytes of one GEMV: packed weight once, activations,
    f32 output."""
    return int(N * K * Q_BYTES[qt]) + M * K * act_bytes + M * N * 4


def profiled_traffic(name):
    """HBM bytes per launch measured by the two rocprofv3 PMC runs
    (FETCH_SIZE, WRITE_SIZE, calibrated on a plain copy) recorded in
    profiles/<name>; None if that summary is absent."""
    import re
    try:
        txt = open(os.path.join(ROOT, "profiles", name)).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", txt)
    return int(m.group(1)) if m else None


def make_weights(qt, N, K, copies, dev, seed=0x5EED):
    """`copies` distinct SoA weights generated on the GPU (random codes and
    bytes, fp16 scales ~ U(0.001, 0.02))."""
    from ubridge_amd import ops
    g = torch.Generator(device=dev).manual_seed(seed)
    nb = N * K // ops.BLOCK[qt]
    out = []
    for _ in range(copies):
        w = torch.randint(0, 256, (ops.quant_bytes(qt, N * K),), dtype=torch.uint8, device=dev,
                          generator=g)
        hb = 16 if qt == 12 else 2
        hdr = w[: nb * hb].view(nb, hb)
        hdr[:, 0:2] = (torch.rand(nb, generator=g, device=dev) * 0.019 + 0.001).half().view(
            torch.uint8).view(nb, 2)
        if qt == 12:
            hdr[:, 2:4] = (torch.rand(nb, generator=g, device=dev) * 0.019 + 0.001).half().view(
                torch.uint8).view(nb, 2)
        if qt == 8:  # int8 codes uniform in -127..127
            q = w[nb * hb:].view(torch.int8)
            q[q == -128] = -127
        out.append(w)
    return out


def time_graph(fn_list, reps, stream, min_calls=60):
    """Capture fn_list (repeated to >= min_calls calls: shorter graphs leave
    a gap between replays) into one HIP graph, replay it untimed for ~0.05 s,
    then time `reps` replays with events on the launch stream.  Returns
    seconds per call."""
    fn_list = list(fn_list) * -(-min_calls // len(fn_list))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for fn in fn_list:
            fn()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):  # replay() launches on the current stream
        t_w = time.perf_counter()
        while time.perf_counter() - t_w < 0.05:
            g.replay()
            torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / 1e3 / (reps * len(fn_list))


def time_eager(fn, reps, stream, warmup=2):
    """Time back-to-back launches of fn on `stream` with HIP events."""
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / 1e3 / reps


def bench_gemv(qt, M, K, N, dev, copies=None, reps=20, x_dtype=torch.bfloat16, full=False):
    """Time the GEMV over rotating weight copies: the kernel alone
    (prequantized activations) or, with full=True, quantize + GEMV.
    Returns (seconds per GEMV, algorithmic bytes)."""
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
    if full:
        fns = [lambda mm=mm: mm.forward(x, out=y, stream=s) for mm in mms]
    else:
        fns = [lambda mm=mm: mm.matmul_prequantized(M, y, stream=s) for mm in mms]
    with torch.cuda.stream(s):
        for fn in fns:
            fn()
    torch.cuda.synchronize()
    t = time_graph(fns, reps, s)
    del ws, mms
    return t, gemv_bytes(qt, M, K, N, 2 if x_dtype == torch.bfloat16 else 4)


def bench_decode_sweep(dev):
    """every Llama-3-8B decode shape (K x N) for Q8_0 and Q4_K at
    M = 1, 4, 16 bf16 tokens.  `step_us` is the whole ubridge_qmatmul call
    (activation quantization + GEMV: one kernel at M = 1, two launches
    above), `gemv_us` the GEMV on activations quantized beforehand; the
    weight rotates over > 512 MB of copies, so both are HBM figures, and
    `pct_hbm_peak` is the step's algorithmic bytes / step time / 8 TB/s."""
    from ubridge_amd import ops
    out = {}
    for sqt in (ops.Q8_0, ops.Q4_K):
        for (sk, sn) in ((4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)):
            for sm in (1, 4, 16):
                t_s, b = bench_gemv(sqt, sm, sk, sn, dev, reps=5, full=True)
                t_g, _ = bench_gemv(sqt, sm, sk, sn, dev, reps=5)
                out[f"{Q_NAME[sqt]}_K{sk}_N{sn}_M{sm}"] = {
                    "step_us": round(t_s * 1e6, 2), "gemv_us": round(t_g * 1e6, 2),
                    "GB/s": round(b / t_s / 1e9, 1),
                    "pct_hbm_peak": round(100 * b / t_s / 1e9 / HBM_PEAK_GBS, 2)}
    return out


def _repeat(fn, seconds):
    """Run fn once untimed, then repeatedly for ~`seconds`; (calls, elapsed)."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            return n, el


def cpu_threads():
    """Threads for the CPU legs: this process's CPU share.  On the GPU boxes
    one GPU's share of the host is OMP_NUM_THREADS (16) cores, whatever the
    host's logical CPU count; elsewhere the CPUs this process may run on."""
    share = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    return min(share, int(omp)) if omp and omp.isdigit() and int(omp) > 0 else share


def cpu_baseline(qt, K, N, seconds, nthreads):
    """Candle-method QMatMul (oracle/ C restatement) on the host cores, one
    bf16-valued token through the full [N, K] weight, repeated for
    ~`seconds`."""
    import numpy as np
    import oracle
    from ubridge_amd import synth
    w = synth.make_weight_soa(qt, N, K, seed=1)
    # the GPU leg's activations are bf16: the same values, held as f32
    x = torch.from_numpy(synth.make_activations(1, K, seed=2)).bfloat16().float().numpy()
    n, el = _repeat(lambda: oracle.qmatmul(qt, w, x, N, K, nthreads), seconds)
    per = el / n
    return {"value": round(gemv_bytes(qt, 1, K, N, 2) / per / 1e9, 3), "unit": "GB/s",
            "cores": nthreads, "kind": "port",
            "host_logical_cpus": os.cpu_count(),
            "sample": f"{n} x one-token Candle-method QMatMul ({Q_NAME[qt]}, K={K}, N={N}, "
                      f"bf16-valued act -> Q8_K, {nthreads} threads) in {el:.1f} s, "
                      f"{per * 1e3:.2f} ms each"}


def cpu_secondary(seconds, nthreads):
    """CPU figures of configs[2]-[4]: the oracle's threaded f32/f64 GEMMs on
    the decoded weights (the restated reference method), each on a bounded
    sample of rows / tokens, scaled to the metric's unit."""
    import numpy as np
    import oracle
    from ubridge_amd import synth
    out = {}
    K, N, G, Ms = 4096, 14336, 128, 64
    qw, sc, qz = synth.make_gptq_w4(K, N, G, seed=2)
    a = synth.bf16_activations(Ms, K, seed=3)
    n, el = _repeat(lambda: oracle.w4a16_gemm(a, qw, sc, qz, Ms, K, N, G, nthreads=nthreads),
                    seconds)
    out["w4a16_prefill"] = {"TFLOP/s": round(2 * Ms * K * N * n / el / 1e12, 5),
                            "sample": f"{n} x M={Ms} rows of configs[2] (int4 dequant + GEMM, "
                                      f"{nthreads} threads) in {el:.1f} s"}
    M, K, N = 16, 8192, 28672
    g = np.random.default_rng(5)
    aq, sa = oracle.fp8_quantize_rows(g.standard_normal((M, K), np.float32))
    wq, sw = oracle.fp8_quantize_rows(g.standard_normal((N, K), np.float32))
    wkn = np.ascontiguousarray(wq.T)
    n, el = _repeat(lambda: oracle.fp8_gemm(aq, sa, wkn, sw, M, K, N, nthreads=nthreads), seconds)
    out["fp8_w8a8"] = {"TFLOP/s": round(2 * M * K * N * n / el / 1e12, 5),
                       "sample": f"{n} x M={M} rows of configs[4] (e4m3 decode + GEMM, "
                                 f"{nthreads} threads) in {el:.1f} s"}
    T, H, E, k, I, bs = 32, 2048, 128, 8, 768, 32
    logits = g.standard_normal((T, E)).astype(np.float32)
    wts, ids = oracle.topk_softmax(logits, k, 1, oracle.F32)
    s_ids, e_ids, ntpp = oracle.moe_align_block_size(ids, E, bs)
    x = synth.f32_to_bf16_bits(g.standard_normal((T, H)).astype(np.float32))
    w13 = g.integers(-127, 128, (E, 2 * I, H), dtype=np.int8)
    s13 = synth.f32_to_bf16_bits(g.uniform(0, 0.002, (E, 2 * I)).astype(np.float32))

    def moe_gate_up():
        oracle.fused_moe(x, None, w13, s13, None, wts.reshape(-1), s_ids, e_ids, ntpp, T, H,
                         2 * I, E, T * k, k, bs, False, nthreads=nthreads)
    n, el = _repeat(moe_gate_up, seconds)
    out["moe_w8a16"] = {"TFLOP/s": round(2 * T * k * H * 2 * I * n / el / 1e12, 5),
                        "sample": f"{n} x gate/up expert GEMM of {T} tokens of configs[3] "
                                  f"(top-{k} of {E}, {nthreads} threads) in {el:.1f} s"}
    return out


def bench_w4a16(dev, Ms=(64, 512, 2048), reps=30):
    from ubridge_amd import ops
    K, N, G = 4096, 14336, 128
    g = torch.Generator(device=dev).manual_seed(3)
    qw = torch.randint(-2**31, 2**31 - 1, (K // 8, N), dtype=torch.int32, device=dev, generator=g)
    sc = (torch.rand(K // G, N, device=dev, generator=g) * 0.018 + 0.002).bfloat16()
    qz = torch.randint(-2**31, 2**31 - 1, (K // G, N // 8), dtype=torch.int32, device=dev,
                       generator=g)
    s = torch.cuda.Stream()
    res = {}
    for M in Ms:
        a = torch.randn(M, K, device=dev, generator=g).bfloat16()
        out = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
        fn = lambda: ops.w4a16_gemm(a, qw, sc, qz, G, out=out, stream=s)
        _eager(fn, s)
        t = time_graph([fn] * 3, max(1, reps // 3), s)
        tf = 2 * M * K * N / t / 1e12
        res[f"M{M}"] = {"us": round(t * 1e6, 1), "TFLOP/s": round(tf, 1),
                        "pct_bf16_mfma_peak": round(100 * tf / BF16_PEAK_TFLOPS, 2),
                        "route": _quant_route(M)}
        if M > 1024:  # the fused kernel at the same size (knob 2: no slab route)
            res[f"M{M}_fused_kernel"] = _fused_leg(fn, s, 2 * M * K * N, reps)
    return {"config": "configs[2]: bf16 A [M, 4096] x GPTQ int4 W [4096, 14336], g=128", **res}


def _fused_leg(fn, s, flop, reps):
    from ubridge_amd import ops
    ops.tune_set("w4a16_path", 2)
    try:
        t = time_graph([fn] * 3, max(1, reps // 3), s)
    finally:
        ops.tune_set("w4a16_path", 0)
    tf = flop / t / 1e12
    return {"us": round(t * 1e6, 1), "TFLOP/s": round(tf, 1),
            "pct_bf16_mfma_peak": round(100 * tf / BF16_PEAK_TFLOPS, 2),
            "route": "pipelined fused-dequant MFMA kernel (w4a16_path = 2)"}


def _eager(fn, s):
    """One eager call on s before capture: the slab route's hipBLASLt plans
    and the stream's workspace are made outside graph capture."""
    with torch.cuda.stream(s):
        fn()
    torch.cuda.synchronize()


def _quant_route(M):
    return ("k_deq_nk (T slab) + hipBLASLt GEMM" if M > 1024
            else "pipelined fused-dequant MFMA kernel, K split over 4 workgroups per tile"
            if M <= 128 else "pipelined fused-dequant MFMA kernel")


def bench_w4_reflayout(dev, Ms=(512, 2048), reps=30):
    """configs[2]'s shape through the reference-named entry point
    matmul_bf16_4bit (uint8 [K/2, N], bf16 scales and zeros, g = 128)."""
    from ubridge_amd import ops
    K, N, G = 4096, 14336, 128
    g = torch.Generator(device=dev).manual_seed(6)
    w = torch.randint(0, 256, (K // 2, N), dtype=torch.uint8, device=dev, generator=g)
    sc = (torch.rand(K // G, N, device=dev, generator=g) * 0.018 + 0.002).bfloat16()
    zr = torch.randint(0, 16, (K // G, N), device=dev, generator=g).bfloat16()
    s = torch.cuda.Stream()
    res = {}
    for M in Ms:
        a = torch.randn(M, K, device=dev, generator=g).bfloat16()
        out = torch.empty(1, M, N, device=dev, dtype=torch.bfloat16)
        fn = lambda: ops.matmul_quant(a, w, sc, zr, bits=4, group_size=G, out=out, stream=s)
        _eager(fn, s)
        t = time_graph([fn] * 3, max(1, reps // 3), s)
        tf = 2 * M * K * N / t / 1e12
        res[f"M{M}"] = {"us": round(t * 1e6, 1), "TFLOP/s": round(tf, 1),
                        "pct_bf16_mfma_peak": round(100 * tf / BF16_PEAK_TFLOPS, 2),
                        "route": _quant_route(M)}
        if M > 1024:
            res[f"M{M}_fused_kernel"] = _fused_leg(fn, s, 2 * M * K * N, reps)
    # decode: one token, the weight rotated over copies totalling > 256 MB so
    # no launch finds it in the MALL; bytes = weight + scales + zeros
    copies = 12
    ws = [torch.randint(0, 256, (K // 2, N), dtype=torch.uint8, device=dev, generator=g)
          for _ in range(copies)]
    a1 = torch.randn(1, K, device=dev, generator=g).bfloat16()
    o1 = torch.empty(1, 1, N, device=dev, dtype=torch.bfloat16)
    fns = [lambda w_=w_: ops.matmul_quant(a1, w_, sc, zr, bits=4, group_size=G, out=o1, stream=s)
           for w_ in ws]
    t = time_graph(fns, max(1, reps // 6), s)
    nbytes = K * N // 2 + 2 * 2 * (K // G) * N
    res["M1"] = {"us": round(t * 1e6, 2), "GB/s": round(nbytes / t / 1e9, 1),
                 "pct_hbm_peak": round(100 * nbytes / t / 1e9 / HBM_PEAK_GBS, 2),
                 "kernel": "k_wq_gemv_os (one-shot direct-to-LDS decode GEMV)"}
    del ws
    return {"config": "configs[2] shape via matmul_bf16_4bit: uint8 [K/2, N] 4-bit, g=128",
            **res}


def bench_fp8(dev, reps=10):
    from ubridge_amd import fp8
    M, K, N = 4096, 8192, 28672
    g = torch.Generator(device=dev).manual_seed(5)
    aq, sa = fp8.quantize_rows(torch.randn(M, K, device=dev, generator=g))
    wq, sw = fp8.quantize_rows(torch.randn(N, K, device=dev, generator=g))  # [N, K] prepacked
    out = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    s = torch.cuda.Stream()
    fn = lambda: fp8.gemm(aq, sa, wq, sw, out=out, stream=s)
    _eager(fn, s)  # the library's hipBLASLt set-up is made outside capture
    t = time_graph([fn] * 2, max(1, reps // 2), s)
    tf = 2 * M * K * N / t / 1e12
    res = {"config": "configs[4]: e4m3 [4096, 8192] x e4m3 [8192, 28672] -> bf16",
           "us": round(t * 1e6, 1), "TFLOP/s": round(tf, 1),
           "pct_fp8_mfma_peak": round(100 * tf / FP8_PEAK_TFLOPS, 2),
           "route": "hipBLASLt fp8 GEMM, row / column f32 scale vectors"}
    from ubridge_amd import ops
    ops.tune_set("gemm_tile", 3)  # the library's own kernel, for comparison
    try:
        t3 = time_graph([fn] * 2, max(1, reps // 2), s)
    finally:
        ops.tune_set("gemm_tile", 0)
    tf3 = 2 * M * K * N / t3 / 1e12
    res["own_kernel"] = {"us": round(t3 * 1e6, 1), "TFLOP/s": round(tf3, 1),
                         "pct_fp8_mfma_peak": round(100 * tf3 / FP8_PEAK_TFLOPS, 2),
                         "route": "k_fp8_gemm2 (gemm_tile = 3)"}
    return res


def bench_moe(dev, reps=20):
    from ubridge_amd import moe
    T, H, E, k, I = 256, 2048, 128, 8, 768
    g = torch.Generator(device=dev).manual_seed(4)
    x = torch.randn(T, H, device=dev, generator=g).bfloat16()
    logits = torch.randn(T, E, device=dev, generator=g).bfloat16()
    w13 = torch.randint(-127, 128, (E, 2 * I, H), device=dev, dtype=torch.int8, generator=g)
    s13 = (torch.rand(E, 2 * I, device=dev, generator=g) * 0.002).bfloat16()
    w2 = torch.randint(-127, 128, (E, H, I), device=dev, dtype=torch.int8, generator=g)
    s2 = (torch.rand(E, H, device=dev, generator=g) * 0.002).bfloat16()
    layer = moe.FusedMoE(w13, w2, s13, s2, topk=k, renormalize=True, block_size=32)
    s = torch.cuda.Stream()
    t = time_graph([lambda: layer(x, logits, stream=s)] * 4, max(1, reps // 4), s)
    wbytes = w13.numel() + w2.numel() + 2 * (s13.numel() + s2.numel())
    flops = 2 * T * k * (H * 2 * I + I * H)
    return {"config": "configs[3]: 256 tok, H=2048, 128 experts, top-8, W8A16 gate/up + down",
            "us": round(t * 1e6, 1), "weight_GB/s": round(wbytes / t / 1e9, 1),
            "pct_hbm_peak": round(100 * wbytes / t / 1e9 / HBM_PEAK_GBS, 2),
            "TFLOP/s": round(flops / t / 1e12, 2)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=600)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run 3 plain 512 MiB device copies (HBM counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU (--gpus {args.gpus} requested): this build's path is "
              "single-GPU (column- / expert-parallel sharding is not built)", file=sys.stderr)
        sys.exit(2)

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
    # timed region: exactly --steps steps, captured as one HIP graph (the
    # weight copies in rotation) and replayed once, HIP events on its stream
    steps = args.steps
    g_t = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_t, stream=s):
        for i in range(steps):
            step(i)
    # untimed replays for ~0.1 s first: clocks settle before the timed region
    with torch.cuda.stream(s):
        t_w = time.perf_counter()
        while time.perf_counter() - t_w < 0.1:
            g_t.replay()
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    with torch.cuda.stream(s):
        # one untimed replay ahead of the first event keeps the GPU busy while
        # the timed replay is submitted (the host's submission latency stays
        # outside the timed region; the ~12 us boundary between two graph
        # replays on this runtime does not, so short --steps pay it once)
        g_t.replay()
        ev[0].record(s)
        g_t.replay()
        ev[1].record(s)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_step = ev[0].elapsed_time(ev[1]) / 1e3 / steps
    algo = gemv_bytes(qt, M, K, N)
    value = algo / per_step / 1e9
    del g_t
    # the roofline figure: median per step over 60 individually timed replays
    # of a graph of `spr` steps (the rotation over the copies, repeated to >=
    # 60 steps: shorter graphs leave a gap between replays that the kernel
    # does not cause)
    spr = copies * -(-60 // copies)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(spr):
            step(i)
    nrep = 60
    ex = [torch.cuda.Event(enable_timing=True) for _ in range(nrep + 1)]
    with torch.cuda.stream(s):
        g.replay()
        ex[0].record(s)
        for i in range(nrep):
            g.replay()
            ex[i + 1].record(s)
    torch.cuda.synchronize()
    samples = [ex[i].elapsed_time(ex[i + 1]) / 1e3 / spr for i in range(nrep)]
    samples.sort()
    med = samples[len(samples) // 2]
    del g, mms, ws

    # ---- roofline of the dominant kernel: the step is one launch of the fused
    # quantize + GEMV kernel, so its HIP-event time per step is the kernel's
    # average duration (graph replay: no host gaps between launches)
    ach = algo / med / 1e9
    roofline = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                "traffic": profiled_traffic("decode_gemv_q4k_4096x28672_hbm_traffic.md"),
                "kernel": "k_gemv_q4k_pq<W=4, MT=1, R=2, out f32, x bf16, NCH=1> "
                          "(persistent grid; Q8_K quantize once per workgroup + GEMV, one kernel)",
                "median_us": round(med * 1e6, 3), "mean_us": round(per_step * 1e6, 3),
                "p10_us": round(samples[len(samples) // 10] * 1e6, 3),
                "p90_us": round(samples[len(samples) * 9 // 10] * 1e6, 3),
                "replays": len(samples), "steps_per_replay": spr, "bytes_per_launch": algo}
    # the GEMV alone, activations quantized beforehand (workspace path)
    t_k, kbytes = bench_gemv(qt, M, K, N, dev, copies=copies, reps=20)
    gemv_pre = {"kernel": "k_gemv_q4k_lds<W=4, MT=1, R=2, out f32> (workspace activations)",
                "us": round(t_k * 1e6, 3), "GB/s": round(kbytes / t_k / 1e9, 1)}

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": steps, "warmup": args.warmup, "ms_per_step": round(per_step * 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded random Q4_K blocks, N(0,1) bf16 activations)",
        "config": {"workload": "decode_gemv q4_k K=4096 N=28672 M=1 (configs[1], Llama-3-8B "
                               "fused gate/up)",
                   "M": M, "K": K, "N": N, "weight_format": "GGUF Q4_K, reference SoA layout",
                   "act_dtype": "bf16",
                   "step": "activation Q8_K quantize + fused GEMV (one kernel)",
                   "weight_copies_rotated": copies,
                   "hbm_pct_of_peak": round(100 * value / HBM_PEAK_GBS, 2),
                   "timed_wall_s": round(wall, 4)},
        "roofline": roofline,
        "gemv_prequantized": gemv_pre,
    }
    if not args.no_secondary:
        sec = {}
        t, b = bench_gemv(ops.Q4_0, 1, 4096, 4096, dev, reps=10, x_dtype=torch.float32, full=True)
        sec["q4_0_gemv_cfg0"] = {"config": "configs[0]: Q4_0 [4096 x 4096], f32 act [1, 4096]",
                                 "us_per_step": round(t * 1e6, 2), "GB/s": round(b / t / 1e9, 1)}
        # configs[0]'s format at 16 bf16 tokens on the Llama-3-8B gate/up
        # shape: Q8_0 quantize launch + the ring GEMV
        t0, b0 = bench_gemv(ops.Q4_0, 16, 4096, 28672, dev, reps=10, full=True)
        sec["q4_0_decode_m16"] = {"config": "Q4_0 K=4096 N=28672, 16 bf16 tokens (ubridge_qmatmul)",
                                  "kernels": "k_quantize_q8_0_v + k_gemv_mm (ring, int8 MFMA)",
                                  "us": round(t0 * 1e6, 2), "GB/s": round(b0 / t0 / 1e9, 1),
                                  "pct_hbm_peak": round(100 * b0 / t0 / 1e9 / HBM_PEAK_GBS, 2)}
        # configs[1] at 16 tokens: the multi-token ring GEMV (workspace
        # activations), and the whole step (Q8_K quantize launch + GEMV)
        t16, b16 = bench_gemv(qt, 16, K, N, dev, reps=10)
        t16f, _ = bench_gemv(qt, 16, K, N, dev, reps=10, full=True)
        sec["q4_k_gemv_m16"] = {"config": "configs[1]: Q4_K K=4096 N=28672, 16 tokens",
                                "kernel": "k_gemv_mm (direct-to-LDS ring, int8 MFMA)",
                                "us": round(t16 * 1e6, 2), "GB/s": round(b16 / t16 / 1e9, 1),
                                "pct_hbm_peak": round(100 * b16 / t16 / 1e9 / HBM_PEAK_GBS, 2),
                                "step_us": round(t16f * 1e6, 2)}
        # QMatMul at prefill size (512 tokens, Q4_K 4096 x 14336): the
        # pipelined MFMA GEMM dequantizing the Q4_K blocks in registers
        tp, _ = bench_gemv(qt, 512, 4096, 14336, dev, reps=4, full=True)
        sec["q4_k_qmatmul_prefill"] = {
            "config": "Q4_K K=4096 N=14336, 512 bf16 tokens (ubridge_qmatmul)",
            "kernels": "k_w4a16<Q4_K> (pipelined GEMM, Q4_K dequantized in registers from LDS)", "us": round(tp * 1e6, 1),
            "TFLOP/s": round(2 * 512 * 4096 * 14336 / tp / 1e12, 1),
            "pct_bf16_mfma_peak": round(100 * 2 * 512 * 4096 * 14336 / tp / 1e12 / BF16_PEAK_TFLOPS, 2)}
        # QMatMul at 64 tokens: the pipelined GEMM with K split over workgroups
        tq, _ = bench_gemv(qt, 64, 4096, 14336, dev, reps=10, full=True)
        sec["q4_k_qmatmul_m64"] = {
            "config": "Q4_K K=4096 N=14336, 64 bf16 tokens (ubridge_qmatmul)",
            "kernels": "k_w4a16<Q4_K> (64-row tiles, K split over 4 workgroups) + k_ksum",
            "us": round(tq * 1e6, 1), "TFLOP/s": round(2 * 64 * 4096 * 14336 / tq / 1e12, 1)}
        sec["w4a16_prefill"] = bench_w4a16(dev)
        sec["matmul_bf16_4bit_prefill"] = bench_w4_reflayout(dev)
        sec["fp8_w8a8"] = bench_fp8(dev)
        sec["moe_w8a16"] = bench_moe(dev)
        sec["decode_sweep_cfg1"] = bench_decode_sweep(dev)
        line["secondary"] = sec
    if args.calibrate_copy:
        src = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        line["calibration_copy_bytes"] = src.numel()
    if not args.no_cpu:
        nthreads = cpu_threads()
        line["cpu_baseline"] = cpu_baseline(qt, K, N, args.cpu_seconds, nthreads)
        if not args.no_secondary:
            line["cpu_baseline"]["secondary"] = cpu_secondary(args.cpu_seconds / 2, nthreads)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
