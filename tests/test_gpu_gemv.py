"""GPU parity of the fused decode GEMV (Candle QMatMul method) against the
CPU oracle.  Integer block dots are exact; only the f32 summation order of
block results differs, so the oracle comparison uses rel-err <= 1e-5 (100x
tighter than the 1e-2 the north star asks of QMatMul output).  At the full
Llama-3-8B shapes the check is against an f64 dense dot of the bit-exact
dequantized weight (activation quantization bounds it by 1e-2)."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from conftest import rel_err
from ubridge_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu


def _run(dev, qt, N, K, x, out_dtype=torch.float32, x_dtype=torch.float32):
    w = synth.make_weight_soa(qt, N, K, seed=N + K + qt)
    mm = ops.QMatMul(qt, torch.from_numpy(w).to(dev), N, K)
    xt = torch.from_numpy(x).to(x_dtype).to(dev)
    y = mm(xt, out_dtype=out_dtype).float().cpu().numpy()
    return w, y


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0, ops.Q4_K])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 16, 17])
def test_gemv_vs_oracle(dev, qt, M):
    N, K = 300, 1536 if qt != ops.Q4_K else 2048
    x = synth.make_activations(M, K, seed=M)
    w, y = _run(dev, qt, N, K, x)
    want = oracle.qmatmul(qt, w, x, N, K)
    assert rel_err(y, want) < 1e-5


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0, ops.Q4_K])
def test_gemv_bf16_in_out(dev, qt):
    N, K, M = 256, 1024, 4
    x = synth.make_activations(M, K, seed=3)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    w, y = _run(dev, qt, N, K, x, out_dtype=torch.bfloat16, x_dtype=torch.bfloat16)
    want = oracle.qmatmul(qt, w, xb.float().numpy(), N, K)
    assert rel_err(y, want) < 4e-3  # bf16 output rounding only


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0, ops.Q4_K])
def test_gemv_exact_activations(dev, qt):
    # lossless activation quantization -> GPU must equal the exact dense dot
    N, K, M = 128, 2048, 2
    g = np.random.default_rng(9)
    x = g.integers(-120, 121, (M, K)).astype(np.float32)
    if qt == ops.Q4_K:
        x.reshape(M, -1, 256)[:, :, 3] = -128.0
    else:
        x.reshape(M, -1, 32)[:, :, 3] = 127.0
    w, y = _run(dev, qt, N, K, x)
    wd = oracle.dequant(qt, w, N * K, oracle.F32).reshape(N, K).astype(np.float64)
    assert rel_err(y, x.astype(np.float64) @ wd.T) < 1e-6


def test_cfg1_q4_0_4096(dev):
    # Q4_0 [4096 x 4096], f32 activations [1, 4096]
    N = K = 4096
    x = synth.make_activations(1, K, seed=0x5EED)
    w, y = _run(dev, ops.Q4_0, N, K, x)
    assert rel_err(y, oracle.qmatmul(ops.Q4_0, w, x, N, K, nthreads=8)) < 1e-5


@pytest.mark.parametrize("qt", [ops.Q8_0, ops.Q4_K, ops.Q4_0])
@pytest.mark.parametrize("K,N", [(8192, 4096), (5120, 14336)])
@pytest.mark.parametrize("M", [2, 3, 4, 6])
def test_decode_routes_off_llama(dev, qt, K, N, M):
    # shapes on either side of the decode route thresholds (rows longer than
    # 8192, matrices of more than 8192 rows): one launch or quantize launch +
    # ring / register GEMV, against the f64 dense dot on the GPU-dequantized
    # weight (activation quantization error only)
    w = synth.make_weight_soa(qt, N, K, seed=K + N + 7)
    wt = torch.from_numpy(w).to(dev)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16)
    print(f"decode route qt={qt} K={K} N={N} M={M}", flush=True)
    y = ops.QMatMul(qt, wt, N, K)(x.to(dev)).double()
    wd = ops.dequantize_block(qt, wt, N * K, torch.float32).view(N, K).double()
    want = x.to(dev).double() @ wd.T
    assert (torch.linalg.norm(y - want) / torch.linalg.norm(want)).item() < 1e-2


@pytest.mark.parametrize("qt", [ops.Q8_0, ops.Q4_K, ops.Q4_0])
@pytest.mark.parametrize("K,N", [(4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)])
@pytest.mark.parametrize("M", [2, 4, 6, 16])
def test_llama_shapes(dev, qt, K, N, M):
    # configs[1] at M = 2, 4, 6 and 16 (one launch, and quantize launch +
    # ring GEMV, by shape and format): against the f64 dense dot on the
    # GPU-dequantized weight (bit-exact with the oracle, checked in
    # test_gpu_quant); then M = 1 with the same bf16 activations (the
    # one-launch kernel of the headline) against the oracle
    w = synth.make_weight_soa(qt, N, K, seed=K + N)
    wt = torch.from_numpy(w).to(dev)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    y = ops.QMatMul(qt, wt, N, K)(x.to(dev)).double()
    wd = ops.dequantize_block(qt, wt, N * K, torch.float32).view(N, K).double()
    want = x.to(dev).double() @ wd.T
    assert (torch.linalg.norm(y - want) / torch.linalg.norm(want)).item() < 1e-2
    if M == 16:
        y1 = ops.QMatMul(qt, wt, N, K)(x[:1].to(dev)).cpu().numpy()
        x1 = x[:1].float().numpy()
        assert rel_err(y1, oracle.qmatmul(qt, w, x1, N, K, nthreads=8)) < 1e-5


def test_activation_workspace_bit_exact(dev):
    # the quantized activations in the workspace equal the oracle's Q8_0 / Q8_K
    K, M = 1024, 3
    x = synth.make_activations(M, K, seed=77)
    from ubridge_amd._lib import lib
    for qt in (ops.Q8_0, ops.Q4_K):
        w = torch.zeros(ops.quant_bytes(qt, 64 * K), dtype=torch.uint8, device=dev)
        mm = ops.QMatMul(qt, w, 64, K)
        mm.quantize(torch.from_numpy(x).to(dev))
        torch.cuda.synchronize()
        ws = mm._ws.cpu().numpy()
        q = ws[: M * K].view(np.int8)
        if qt == ops.Q8_0:
            soa = np.concatenate([oracle.quantize_q8_0(x[m]) for m in range(M)])
            nb = K // 32
            want_q = np.concatenate([oracle.quantize_q8_0(x[m])[2 * nb:] for m in range(M)])
            assert np.array_equal(q, want_q.view(np.int8))
            del soa
        else:
            d, qk, bs = oracle.quantize_q8_k(x)
            assert np.array_equal(q, qk)
    assert lib is not None


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,K", [(3, 1024), (16, 4096), (5, 14336)])
def test_q8_0_workspace_quantize_exact(dev, xdt, M, K):
    # the GEMV workspace's Q8_0 activations (8 lanes per block for 16-byte
    # aligned x, one lane per block otherwise): codes, f32 of the fp16 d and
    # the first-16 code sums equal the oracle's quantize_block_q8_0, aligned
    # and misaligned x alike
    x = synth.make_activations(M, K, seed=M * 31 + K)
    xr = torch.from_numpy(x).to(xdt)
    nb = M * K // 32
    al = lambda n: (n + 255) // 256 * 256
    soa = np.concatenate([oracle.quantize_q8_0(xr[m].float().numpy()) for m in range(M)])
    d_want = np.concatenate([oracle.quantize_q8_0(xr[m].float().numpy())[:2 * (K // 32)]
                             .view(np.float16) for m in range(M)]).astype(np.float32)
    q_want = np.concatenate([oracle.quantize_q8_0(xr[m].float().numpy())[2 * (K // 32):]
                             for m in range(M)]).view(np.int8)
    s_want = q_want.reshape(nb, 32)[:, :16].astype(np.int32).sum(1)
    del soa
    w = torch.zeros(ops.quant_bytes(ops.Q8_0, 64 * K), dtype=torch.uint8, device=dev)
    mm = ops.QMatMul(ops.Q8_0, w, 64, K)
    for shift in (0, 1):  # 16-byte aligned, then misaligned by one element
        buf = torch.zeros(M * K + 16, dtype=xdt, device=dev)
        xd = buf[shift:shift + M * K].view(M, K)
        xd.copy_(xr.to(dev))
        assert (xd.data_ptr() % 16 == 0) == (shift == 0)
        mm.quantize(xd)
        torch.cuda.synchronize()
        ws = mm._ws.cpu().numpy()
        assert np.array_equal(ws[:M * K].view(np.int8), q_want), shift
        d = ws[al(M * K):al(M * K) + 4 * nb].view(np.float32)
        sm = ws[al(M * K) + al(4 * nb):al(M * K) + al(4 * nb) + 4 * nb].view(np.int32)
        assert np.array_equal(d, d_want), shift
        assert np.array_equal(sm, s_want), shift


def test_gemv_m0_and_k0(dev):
    w = torch.zeros(ops.quant_bytes(ops.Q8_0, 64 * 32), dtype=torch.uint8, device=dev)
    mm = ops.QMatMul(ops.Q8_0, w, 64, 32)
    y = mm(torch.zeros(0, 32, device=dev))
    assert y.shape == (0, 64)


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("K,N", [(2048, 300), (5120, 77), (4096, 1000), (4096, 28672)])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_q4k_fused_quantize_matches_two_launch(dev, M, K, N, xdt):
    # ubridge_qmatmul quantizes Q4_K activations inside the GEMV kernel for
    # M <= 4; the result must equal quantize-then-GEMV bit for bit where that
    # runs the same kernel family (and to f32 summation order where the
    # two-launch form takes the ring GEMV), and the oracle to the
    # summation-order tolerance.
    x = synth.make_activations(M, K, seed=K + N + M)
    w = synth.make_weight_soa(ops.Q4_K, N, K, seed=N)
    mm = ops.QMatMul(ops.Q4_K, torch.from_numpy(w).to(dev), N, K)
    xt = torch.from_numpy(x).to(dev).to(xdt)
    fused = mm(xt).cpu().numpy()
    mm.quantize(xt)
    two = torch.empty(M, N, device=dev)
    mm.matmul_prequantized(M, two)
    if M <= 2 or N < 16384:
        assert np.array_equal(fused, two.cpu().numpy())
    else:
        assert rel_err(fused, two.cpu().numpy()) < 1e-6
    want = oracle.qmatmul(ops.Q4_K, w, xt.float().cpu().numpy(), N, K, nthreads=8)
    assert rel_err(fused, want) < 1e-5


@pytest.mark.parametrize("qt", [ops.Q8_0, ops.Q4_K])
@pytest.mark.parametrize("M", [2, 3, 8, 16, 17])
def test_gemv_mfma_path_vs_oracle(dev, qt, M):
    # the int8-MFMA multi-token GEMV, forced on from M = 2 (gemv_mfma_m knob);
    # K spans a partial 512-element chunk and more chunks than wavefronts
    N, K = 88, 9216 + (256 if qt == ops.Q4_K else 160)  # N*K/32*2 % 16 == 0 (Q8_0 payload alignment)
    old = ops.tune_get("gemv_mfma_m")
    ops.tune_set("gemv_mfma_m", 2)
    ops.tune_set("w4a16_path", 2)  # M = 17 stays on the GEMV (not the prefill GEMM)
    try:
        x = synth.make_activations(M, K, seed=M + 5)
        w, y = _run(dev, qt, N, K, x)
    finally:
        ops.tune_set("gemv_mfma_m", old)
        ops.tune_set("w4a16_path", 0)
    assert rel_err(y, oracle.qmatmul(qt, w, x, N, K)) < 1e-5


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0, ops.Q4_K])
@pytest.mark.parametrize("cfg", list(range(1, 23)))
@pytest.mark.parametrize("M,K,N", [(3, 3072, 200), (7, 1024, 77), (16, 6144, 130), (17, 2048, 64), (4, 4096, 16400)])
def test_gemv_ring_vs_oracle(dev, qt, cfg, M, K, N):
    # the direct-to-LDS ring GEMV (3..16 tokens, K % 1024 == 0; Q4_0 / Q8_0
    # at 3-4 tokens take the one-launch kernel instead), every
    # variant (gemv_mm knob; 22 = the any-K fallback variant): partial row
    # tiles, fewer K steps than ring stages, unused token slots, K the
    # variant's step does not divide, and M = 17 (a 16-token and a 1-token
    # pass)
    old = ops.tune_get("gemv_mm")
    ops.tune_set("gemv_mm", cfg)
    ops.tune_set("w4a16_path", 2)  # M = 17 stays on the GEMV (not the prefill GEMM)
    try:
        x = synth.make_activations(M, K, seed=M + cfg)
        w, y = _run(dev, qt, N, K, x)
    finally:
        ops.tune_set("gemv_mm", old)
        ops.tune_set("w4a16_path", 0)
    assert rel_err(y, oracle.qmatmul(qt, w, x, N, K)) < 1e-5


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0, ops.Q4_K])
@pytest.mark.parametrize("N", [50, 6144, 20000])
@pytest.mark.parametrize("K", [2048, 4096])
def test_gemv_ring_exact_activations(dev, qt, N, K):
    # the ring GEMV's default variant per width (N >= 16384: 112-row tiles;
    # 4096 < N: 32-row tiles; else 16-row tiles), 16 tokens with losslessly
    # quantizable activations: the GPU result must equal the exact dense dot
    # of the dequantized weight (only f32 summation order differs).  K = 4096
    # fills the wide variants' per-row header capacity (16 super-blocks), the
    # case where the header load's last instruction is only partly in range.
    M = 16
    g = np.random.default_rng(N)
    x = g.integers(-120, 121, (M, K)).astype(np.float32)
    if qt == ops.Q4_K:
        x.reshape(M, -1, 256)[:, :, 3] = -128.0
    else:
        x.reshape(M, -1, 32)[:, :, 3] = 127.0
    w, y = _run(dev, qt, N, K, x)
    wd = oracle.dequant(qt, w, N * K, oracle.F32).reshape(N, K).astype(np.float64)
    assert rel_err(y, x.astype(np.float64) @ wd.T) < 1e-6


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0, ops.Q4_K])
def test_gemv_ring_bf16_in_out(dev, qt):
    N, K, M = 300, 3072, 12
    x = synth.make_activations(M, K, seed=12)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    w, y = _run(dev, qt, N, K, x, out_dtype=torch.bfloat16, x_dtype=torch.bfloat16)
    want = oracle.qmatmul(qt, w, xb.float().numpy(), N, K)
    assert rel_err(y, want) < 4e-3  # bf16 output rounding only


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0])
@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("K,N", [(8192, 77), (1024, 300)])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,iters", [(0, 0), (1, 1), (4, 0)])
def test_q80_fused_quantize_vs_oracle(dev, qt, M, K, N, xdt, rows, iters):
    # one-launch QMatMul for Q4_0 / Q8_0 (the GEMV quantizes x itself): K up
    # to its 8192 limit, a partial last workgroup, every rows / iterations shape
    x = synth.make_activations(M, K, seed=K + M)
    xr = torch.from_numpy(x).to(xdt)
    old = ops.tune_get("gemv_rows"), ops.tune_get("gemv_iters")
    ops.tune_set("gemv_rows", rows)
    ops.tune_set("gemv_iters", iters)
    try:
        w, y = _run(dev, qt, N, K, x, x_dtype=xdt)
    finally:
        ops.tune_set("gemv_rows", old[0])
        ops.tune_set("gemv_iters", old[1])
    assert rel_err(y, oracle.qmatmul(qt, w, xr.float().numpy(), N, K)) < 1e-5


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M", [1, 2])
def test_q4k_fused_quantizer_matches_workspace_quantizer(dev, x_dtype, M, waves):
    # The one-call Q4_K kernel quantizes activations in every workgroup; with
    # the same launch shape it must give bit-identical outputs to the
    # prequantized kernel fed by ubridge_quantize_activations (itself pinned
    # bit-exact to the oracle).  Blocks with +a and -a both at the largest
    # |x| (lowest index decides), all-zero blocks, and values landing exactly
    # on .5 after scaling (round half away from zero) are included.
    N, K = 384, 4096
    g = np.random.default_rng(11 + M)
    x = g.standard_normal((M, K)).astype(np.float32)
    xb = x.reshape(M, -1, 256)
    xb[:, 1, :] = 0.0                                   # zero block
    xb[:, 2, 7], xb[:, 2, 3] = 5.0, -5.0                # tie, negative first
    xb[:, 3, 3], xb[:, 3, 9] = 4.0, -4.0                # tie, positive first
    xb[:, 4, :] = (g.integers(-255, 256, 256) / 2.0)    # iscale -1/-0.5..: .5 steps
    xb[:, 4, 0] = -128.0
    xb[:, 5, :] = g.integers(-3, 4, 256).astype(np.float32) * 0.5
    xb[:, 5, 10] = 2.0
    if x_dtype == torch.bfloat16:
        x = torch.from_numpy(x).bfloat16().float().numpy()
    w = synth.make_weight_soa(ops.Q4_K, N, K, seed=5)
    mm = ops.QMatMul(ops.Q4_K, torch.from_numpy(w).to(dev), N, K)
    xt = torch.from_numpy(x).to(x_dtype).to(dev)
    ops.tune_set("gemv_lds_rows", 2)
    ops.tune_set("gemv_lds_waves", waves)
    try:
        fused = mm(xt).cpu()
        Mq = mm.quantize(xt)
        pre = torch.empty(M, N, device=dev)
        mm.matmul_prequantized(Mq, pre)
        pre = pre.cpu()
    finally:
        ops.tune_set("gemv_lds_rows", 0)
        ops.tune_set("gemv_lds_waves", 0)
    assert torch.equal(fused.view(torch.int32), pre.view(torch.int32))
    assert rel_err(fused.numpy(), oracle.qmatmul(ops.Q4_K, w, x, N, K)) < 1e-5


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0, ops.Q4_K])
@pytest.mark.parametrize("M", [1, 2])
def test_qmatmul_misaligned_x(dev, qt, M):
    # x not 16-byte aligned: the one-launch kernels need 16-byte loads, so the
    # call takes the quantize + GEMV launches instead, with the same result
    N, K = 200, 2048
    x = synth.make_activations(M, K, seed=31)
    w = synth.make_weight_soa(qt, N, K, seed=31)
    mm = ops.QMatMul(qt, torch.from_numpy(w).to(dev), N, K)
    buf = torch.zeros(M * K + 1, device=dev)
    buf[1:] = torch.from_numpy(x).reshape(-1).to(dev)
    xm = buf[1:].view(M, K)
    assert xm.data_ptr() % 16 == 4
    got = mm(xm).cpu().numpy()
    # the same as quantize + GEMV launches on aligned x (the one-launch
    # kernels may sum blocks in another order: both within 1e-5 of the oracle)
    mm.quantize(torch.from_numpy(x).to(dev))
    two = torch.empty(M, N, device=dev)
    mm.matmul_prequantized(M, two)
    assert np.array_equal(got, two.cpu().numpy())
    want = oracle.qmatmul(qt, w, x, N, K)
    assert rel_err(got, want) < 1e-5
    assert rel_err(mm(torch.from_numpy(x).to(dev)).cpu().numpy(), want) < 1e-5


@pytest.mark.parametrize("M,K,N", [(m, k, n) for m in (1, 2, 3, 4)
                                   for k, n in ((4096, 20003), (2048, 300), (5120, 77),
                                                (4096, 28672), (12288, 9000))
                                   if m <= 2 or k <= 4096])  # one launch: <= 2 tokens past K = 4096
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_q4k_persistent_matches_one_shot(dev, M, K, N, xdt):
    # the persistent one-launch Q4_K GEMV (x quantized once per workgroup,
    # row groups looped over a resident grid), with and without the rolling
    # prefetch (gemv_persist 3 / 2), against the one-shot grid: the same
    # arithmetic, so bit-identical; rows past N in the last row group, K over
    # several chunks, and N large enough that workgroups loop
    x = synth.make_activations(M, K, seed=K + M)
    w = synth.make_weight_soa(ops.Q4_K, N, K, seed=N % 1000)
    mm = ops.QMatMul(ops.Q4_K, torch.from_numpy(w).to(dev), N, K)
    xt = torch.from_numpy(x).to(dev).to(xdt)
    old = ops.tune_get("gemv_persist")
    got = {}
    try:
        for mode in (-1, 1, 2, 3, 0):
            ops.tune_set("gemv_persist", mode)
            got[mode] = mm(xt).cpu()
    finally:
        ops.tune_set("gemv_persist", old)
    one = got[-1]
    for mode in (1, 2, 3, 0):
        assert torch.equal(one.view(torch.int32), got[mode].view(torch.int32)), mode
    per = got[1]
    if N <= 9000:
        want = oracle.qmatmul(ops.Q4_K, w, xt.float().cpu().numpy(), N, K, nthreads=8)
        assert rel_err(per.numpy(), want) < 1e-5


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("K,N", [(4096, 4096), (14336, 300), (5120, 77), (256, 1000)])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,waves", [(0, 0), (1, 8), (4, 4)])
def test_q80_lds_one_launch_vs_oracle(dev, qt, M, K, N, xdt, rows, waves):
    # the LDS-staged one-launch Q4_0 / Q8_0 GEMV (activations quantized to
    # Q8_0 once per workgroup): K over one to four 4096-element chunks (the
    # last partial), partial row groups, each wavefront / row shape; the same
    # numbers as the register path up to f32 summation order
    x = synth.make_activations(M, K, seed=K + M + N)
    xr = torch.from_numpy(x).to(xdt)
    w = synth.make_weight_soa(qt, N, K, seed=N + qt)
    mm = ops.QMatMul(qt, torch.from_numpy(w).to(dev), N, K)
    old = ops.tune_get("gemv_lds_rows"), ops.tune_get("gemv_lds_waves")
    ops.tune_set("gemv_lds_rows", rows)
    ops.tune_set("gemv_lds_waves", waves)
    try:
        y = mm(xr.to(dev)).cpu().numpy()
    finally:
        ops.tune_set("gemv_lds_rows", old[0])
        ops.tune_set("gemv_lds_waves", old[1])
    want = oracle.qmatmul(qt, w, xr.float().numpy(), N, K, nthreads=8)
    assert rel_err(y, want) < 1e-5


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0])
@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("K,N", [(4096, 28672), (14336, 4096), (4096, 20003), (12288, 300)])
def test_q80_lds_rolling_prefetch(dev, qt, M, K, N):
    # the one-launch Q4_0 / Q8_0 GEMV with and without the rolling prefetch
    # (gemv_persist 3 / 2): bit-identical (the same arithmetic in the same
    # order), and against the oracle; wide grids whose workgroups loop over
    # row groups, several chunks per row, a partial last row group
    x = synth.make_activations(M, K, seed=K + M + N)
    w = synth.make_weight_soa(qt, N, K, seed=N + qt)
    mm = ops.QMatMul(qt, torch.from_numpy(w).to(dev), N, K)
    xt = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    old = ops.tune_get("gemv_persist")
    got = {}
    try:
        for mode in (2, 3, 0):
            ops.tune_set("gemv_persist", mode)
            got[mode] = mm(xt).cpu()
    finally:
        ops.tune_set("gemv_persist", old)
    assert torch.equal(got[2].view(torch.int32), got[3].view(torch.int32))
    assert torch.equal(got[2].view(torch.int32), got[0].view(torch.int32))
    want = oracle.qmatmul(qt, w, xt.float().cpu().numpy(), N, K, nthreads=8)
    assert rel_err(got[3].numpy(), want) < 1e-5


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0])
def test_q80_lds_exact_activations(dev, qt):
    # losslessly quantizable activations (integers, 127 in every block): the
    # LDS path equals the exact dense dot of the dequantized weight
    N, K, M = 130, 8192, 2
    g = np.random.default_rng(3)
    x = g.integers(-120, 121, (M, K)).astype(np.float32)
    x.reshape(M, -1, 32)[:, :, 5] = 127.0
    w = synth.make_weight_soa(qt, N, K, seed=5)
    y = ops.QMatMul(qt, torch.from_numpy(w).to(dev), N, K)(torch.from_numpy(x).to(dev)).cpu().numpy()
    wd = oracle.dequant(qt, w, N * K, oracle.F32).reshape(N, K).astype(np.float64)
    assert rel_err(y, x.astype(np.float64) @ wd.T) < 1e-6


# ---- QMatMul from 64 tokens on: the reference's GCU sequence (dequantize,
# bf16 GEMM) -- Q4_K by the pipelined GEMM dequantizing in registers, slabs
# through hipBLASLt, or one GEMM dequantizing into LDS

@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0, ops.Q4_K])
@pytest.mark.parametrize("M,K,N", [(128, 1024, 200), (200, 2048, 516), (300, 512, 1024)])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
def test_qmatmul_prefill_gemm(dev, qt, M, K, N, xdt):
    # default (Q4_K: the pipelined GEMM where N % 8 == 0; else hipBLASLt on
    # dequantized slabs): GEMM tolerance of the same
    # products; knob w4a16_path = 1 (the MFMA core dequantizing into LDS):
    # bit-equal to dequantize_block_*_bf16 + ubridge_gemm_dense; both within
    # GEMM tolerance of the f64 product of the oracle's dequantization
    w = synth.make_weight_soa(qt, N, K, seed=M + K + N)
    wt = torch.from_numpy(w).to(dev)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).to(xdt).to(dev)
    mm = ops.QMatMul(qt, wt, N, K)
    wd = ops.dequantize_block(qt, wt, N * K, torch.bfloat16).view(N, K)
    ref = ops.gemm_dense(x.to(torch.bfloat16), wd, w_transposed=True)
    y32 = mm(x)
    y16 = mm(x, out_dtype=torch.bfloat16)
    assert ((y32.double() - ref.double()).norm() / ref.double().norm()).item() < 4e-3
    assert ((y16.double() - ref.double()).norm() / ref.double().norm()).item() < 4e-3
    ops.tune_set("w4a16_path", 1)
    try:
        l32 = mm(x)
        l16 = mm(x, out_dtype=torch.bfloat16)
    finally:
        ops.tune_set("w4a16_path", 0)
    assert torch.equal(l16.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(l32.to(torch.bfloat16).view(torch.int16), ref.view(torch.int16))
    wo = oracle.dequant(qt, w, N * K, oracle.F32).reshape(N, K).astype(np.float64)
    want = x.to(torch.bfloat16).double().cpu().numpy() @ wo.T
    assert rel_err(y32.double().cpu().numpy(), want) < 1e-2


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0, ops.Q4_K])
@pytest.mark.parametrize("M,K,N", [(64, 256, 8), (100, 1024, 264), (512, 4096, 1024),
                                   (777, 2048, 776), (1200, 512, 2056)])
def test_qmatmul_fused_gemm(dev, qt, M, K, N):
    # the pipelined GEMM dequantizing GGUF blocks in registers (knob
    # w4a16_path = 4; by default below 768 tokens), split over K or not
    # by the shape rule; N = 8 / 264 / 776 cut column tiles.  The same bf16
    # weights as dequantize_block_*_bf16 + ubridge_gemm_dense, f32 sums in
    # another order: GEMM tolerance, most bf16 outputs identical; and within
    # GEMM tolerance of the slab route (knob 2) and the f64 oracle
    w = synth.make_weight_soa(qt, N, K, seed=M + N)
    wt = torch.from_numpy(w).to(dev)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(K)).to(torch.bfloat16).to(dev)
    mm = ops.QMatMul(qt, wt, N, K)
    wd = ops.dequantize_block(qt, wt, N * K, torch.bfloat16).view(N, K)
    ref = ops.gemm_dense(x, wd, w_transposed=True)
    ops.tune_set("w4a16_path", 4)  # the pipelined GEMM at every size
    try:
        y32 = mm(x)
        y16 = mm(x, out_dtype=torch.bfloat16)
    finally:
        ops.tune_set("w4a16_path", 0)
    for y in (y32, y16):
        assert ((y.double() - ref.double()).norm() / ref.double().norm()).item() < 4e-3
    assert (y16 == ref).float().mean().item() > 0.9
    ops.tune_set("w4a16_path", 2)
    try:
        s32 = mm(x)
    finally:
        ops.tune_set("w4a16_path", 0)
    assert ((y32.double() - s32.double()).norm() / s32.double().norm()).item() < 4e-3
    wo = oracle.dequant(qt, w, N * K, oracle.F32).reshape(N, K).astype(np.float64)
    want = x.double().cpu().numpy() @ wo.T
    assert rel_err(y32.double().cpu().numpy(), want) < 1e-2


def test_qmatmul_gemm_threshold(dev):
    # Q4_K on a narrow matrix (N < 8192): 39 tokens stay on the GEMV (the
    # Candle method, against the oracle at 1e-5); 40 take the reference's
    # sequence (bf16 activations, ~1e-3 off); Q4_0 on a wide one from 17
    qt, K, N = ops.Q4_K, 1024, 256
    w = synth.make_weight_soa(qt, N, K, seed=5)
    x = synth.make_activations(64, K, seed=5)
    mm = ops.QMatMul(qt, torch.from_numpy(w).to(dev), N, K)
    y39 = mm(torch.from_numpy(x[:39]).to(dev)).cpu().numpy()
    assert rel_err(y39, oracle.qmatmul(qt, w, x[:39], N, K)) < 1e-5
    y40 = mm(torch.from_numpy(x[:40]).to(dev)).cpu().numpy()
    e = rel_err(y40, oracle.qmatmul(qt, w, x[:40], N, K))
    assert 1e-5 < e < 1e-2
    qt, K, N = ops.Q4_0, 256, 8192
    w = synth.make_weight_soa(qt, N, K, seed=6)
    x = synth.make_activations(17, K, seed=6)
    mm = ops.QMatMul(qt, torch.from_numpy(w).to(dev), N, K)
    y16 = mm(torch.from_numpy(x[:16]).to(dev)).cpu().numpy()
    assert rel_err(y16, oracle.qmatmul(qt, w, x[:16], N, K)) < 1e-5
    y17 = mm(torch.from_numpy(x).to(dev)).cpu().numpy()
    e = rel_err(y17, oracle.qmatmul(qt, w, x, N, K))
    assert 1e-5 < e < 1e-2


def test_qmatmul_slabs(dev):
    # a weight larger than one 256 MB bf16 slab (16384 rows at K = 8192): a
    # full slab and a partial one, against the single dense product
    qt, M, K, N = ops.Q8_0, 64, 8192, 16500
    w = synth.make_weight_soa(qt, N, K, seed=9)
    wt = torch.from_numpy(w).to(dev)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).to(dev)
    y = ops.QMatMul(qt, wt, N, K)(x)
    wd = ops.dequantize_block(qt, wt, N * K, torch.bfloat16).view(N, K)
    ref = ops.gemm_dense(x, wd, w_transposed=True)
    assert ((y.double() - ref.double()).norm() / ref.double().norm()).item() < 4e-3


def _misaligned_bf16(x_np, dev):
    """bf16 device copy of x whose data pointer is 2 bytes past 16-byte
    alignment (a view into a larger buffer)."""
    t = torch.from_numpy(x_np).to(dev).to(torch.bfloat16)
    buf = torch.zeros(t.numel() + 1, dtype=torch.bfloat16, device=dev)
    buf[1:] = t.reshape(-1)
    xm = buf[1:].view(t.shape)
    assert xm.data_ptr() % 16 == 2
    return xm, t


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0, ops.Q4_K])
@pytest.mark.parametrize("M", [64, 512])
def test_qmatmul_misaligned_bf16_x_gemm_sizes(dev, qt, M):
    # at GEMM sizes the routes read x rows with 16-byte (direct-to-LDS) loads:
    # a misaligned bf16 x is copied into the workspace first, so the result is
    # bit-identical to the aligned call -- for ubridge_qmatmul and for the
    # allocation-free entry point
    N, K = 520, 1024
    x = synth.make_activations(M, K, seed=M + qt)
    w = torch.from_numpy(synth.make_weight_soa(qt, N, K, seed=qt)).to(dev)
    mm = ops.QMatMul(qt, w, N, K)
    xm, xa = _misaligned_bf16(x, dev)
    print(f"misaligned qmatmul qt={qt} M={M}", flush=True)
    got = mm(xm).cpu().numpy()
    ref = mm(xa).cpu().numpy()
    assert np.array_equal(got, ref)
    noalloc = _lib.register("ubridge_qmatmul_noalloc", ctypes.c_int,
                            [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                             ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                             ctypes.c_int, ctypes.c_void_p])
    y = torch.full((M, N), float("nan"), device=dev)
    y2 = torch.full((M, N), float("nan"), device=dev)
    s = torch.cuda.current_stream().cuda_stream
    _lib.check(noalloc(qt, w.data_ptr(), xm.data_ptr(), ops.BF16, y.data_ptr(), 0, M, N, K, s))
    _lib.check(noalloc(qt, w.data_ptr(), xa.data_ptr(), ops.BF16, y2.data_ptr(), 0, M, N, K, s))
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    xf = torch.from_numpy(x).to(dev).to(torch.bfloat16).float().cpu().numpy()
    assert rel_err(got, oracle.qmatmul(qt, synth.make_weight_soa(qt, N, K, seed=qt), xf, N, K)) < 1e-2
