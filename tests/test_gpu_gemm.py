"""GPU parity of the MFMA GEMM family against the CPU oracle.

W4A16 / W8A16 / dense outputs are bf16 of an f32 MFMA accumulation; the
oracle accumulates in f64 and rounds once, so outputs agree to bf16
rounding: the test bound is rel-err (Frobenius) <= 1e-2 as the north star
states, and in practice ~1e-3.  Dequantized weights are bit-exact."""
import numpy as np
import pytest
import torch

import oracle
from conftest import rel_err
from ubridge_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu


def _bf(x):  # uint16 bits -> torch bf16 on the GPU
    return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).view(torch.bfloat16).cuda()


def _np(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("M,K,N,group", [(64, 256, 128, 128), (130, 512, 264, 128), (1, 128, 8, 32),
                                         (257, 1024, 384, 64), (33, 200, 96, 40)])
def test_w4a16_vs_oracle(dev, M, K, N, group):
    qw, sc, qz = synth.make_gptq_w4(K, N, group, seed=M + N)
    a = synth.bf16_activations(M, K, seed=K)
    out = ops.w4a16_gemm(_bf(a), torch.from_numpy(qw).cuda(), _bf(sc), torch.from_numpy(qz).cuda(),
                         group)
    want = oracle.w4a16_gemm(a, qw, sc, qz, M, K, N, group, nthreads=8)
    err = rel_err(oracle.bf16_to_f32(_np(out)), oracle.bf16_to_f32(want))
    assert err < 1e-2, err
    # bf16 rounding of an f32 vs f64 accumulation: nearly all outputs identical
    # (up to 16 tokens the decode GEMV scales the unrounded weight instead:
    # its exactness check is test_w4a16_decode_gemv)
    if M > 16:
        assert np.mean(_np(out) == want) > 0.9


@pytest.mark.parametrize("tile", [1, 3])  # 128 x 256 split-K / 256 x 256
@pytest.mark.parametrize("M,K,N,group", [(300, 1152, 520, 128), (77, 384, 264, 64),
                                         (256, 4096, 512, 128)])
def test_w4a16_tiles(dev, tile, M, K, N, group):
    qw, sc, qz = synth.make_gptq_w4(K, N, group, seed=M + K)
    a = synth.bf16_activations(M, K, seed=N)
    ops.tune_set("gemm_tile", tile)
    try:
        out = ops.w4a16_gemm(_bf(a), torch.from_numpy(qw).cuda(), _bf(sc),
                             torch.from_numpy(qz).cuda(), group)
    finally:
        ops.tune_set("gemm_tile", 0)
    want = oracle.w4a16_gemm(a, qw, sc, qz, M, K, N, group, nthreads=8)
    err = rel_err(oracle.bf16_to_f32(_np(out)), oracle.bf16_to_f32(want))
    assert err < 1e-2, err
    assert np.mean(_np(out) == want) > 0.9


@pytest.mark.parametrize("M,path", [(512, 0), (2048, 0), (2048, 2)])
def test_w4a16_cfg3(dev, M, path):
    # configs[2] at M = 512 and 2048 on the default route (the pipelined
    # kernel at 512, dequantized slabs + hipBLASLt at 2048) and, at 2048, on
    # the pipelined kernel forced by the w4a16_path = 2 knob (256x256 tiles,
    # 448 of them): against an f64 GPU matmul of the oracle's bit-exact
    # dequant, also per 256-row band so a misplaced tile cannot hide in the
    # global norm
    K, N, group = 4096, 14336, 128
    qw, sc, qz = synth.make_gptq_w4(K, N, group, seed=2)
    a = synth.bf16_activations(M, K, seed=3)
    ops.tune_set("w4a16_path", path)
    try:
        out = ops.w4a16_gemm(_bf(a), torch.from_numpy(qw).cuda(), _bf(sc),
                             torch.from_numpy(qz).cuda(), group)
    finally:
        ops.tune_set("w4a16_path", 0)
    wd = torch.from_numpy(oracle.bf16_to_f32(oracle.w4a16_dequant(qw, sc, qz, K, N, group))).cuda()
    want = _bf(a).double() @ wd.double()
    err = (torch.linalg.norm(out.double() - want) / torch.linalg.norm(want)).item()
    assert err < 1e-2, err
    band = [(torch.linalg.norm(out[i:i + 256].double() - want[i:i + 256]) /
             torch.linalg.norm(want[i:i + 256])).item() for i in range(0, M, 256)]
    assert max(band) < 1e-2, band


@pytest.mark.parametrize("rhs_t", [0, 1])
@pytest.mark.parametrize("group", [-1, 128])
@pytest.mark.parametrize("M,K,N", [(48, 256, 192), (129, 384, 132)])
def test_matmul_bf16_8bit(dev, rhs_t, group, M, K, N):
    g = np.random.default_rng(M * K + N)
    w = g.integers(-127, 128, (N, K) if rhs_t else (K, N)).astype(np.int8)
    ng = 1 if group == -1 else -(-K // group)
    sc = synth.f32_to_bf16_bits(g.uniform(0.002, 0.02, (ng, N)).astype(np.float32))
    a = synth.bf16_activations(M, K, seed=5)
    out = ops.matmul_quant(_bf(a), torch.from_numpy(w).cuda(), _bf(sc), bits=8, group_size=group,
                           rhs_transpose=bool(rhs_t))
    want = oracle.w8a16_gemm(a, w, sc, M, K, N, group, rhs_t)
    assert rel_err(oracle.bf16_to_f32(_np(out)), oracle.bf16_to_f32(want)) < 1e-2


def test_matmul_bf16_4bit_reference_layout(dev):
    M, K, N, group = 70, 256, 128, 64
    g = np.random.default_rng(11)
    rhs = g.integers(0, 256, (K // 2, N)).astype(np.uint8)
    sc = synth.f32_to_bf16_bits(g.uniform(0.002, 0.02, (K // group, N)).astype(np.float32))
    zr = synth.f32_to_bf16_bits(g.integers(0, 16, (K // group, N)).astype(np.float32) + 0.5)
    a = synth.bf16_activations(M, K, seed=6)
    out = ops.matmul_quant(_bf(a), torch.from_numpy(rhs).cuda(), _bf(sc), _bf(zr), bits=4,
                           group_size=group)
    wd = oracle.dequant_u4_ref(rhs, sc, zr, K // 2, N, group, oracle.BF16)
    want = oracle.bf16_to_f32(a).astype(np.float64) @ oracle.bf16_to_f32(wd).astype(np.float64)
    assert rel_err(oracle.bf16_to_f32(_np(out)), want) < 1e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dequant_u4_bit_exact(dev, dtype):
    K, N, group = 96, 64, 64  # K packed rows -> 192 weight rows
    g = np.random.default_rng(1)
    rhs = g.integers(0, 256, (K, N)).astype(np.uint8)
    sc32 = g.uniform(0.002, 0.02, (2 * K // group, N)).astype(np.float32)
    z32 = (g.integers(0, 16, (2 * K // group, N)) + 0.25).astype(np.float32)
    if dtype == torch.bfloat16:
        sc, zr, dt = synth.f32_to_bf16_bits(sc32), synth.f32_to_bf16_bits(z32), oracle.BF16
        st, zt = _bf(sc), _bf(zr)
    else:
        sc, zr, dt = sc32.astype(np.float16).view(np.uint16), z32.astype(np.float16).view(np.uint16), oracle.F16
        st = torch.from_numpy(sc.view(np.float16)).cuda()
        zt = torch.from_numpy(zr.view(np.float16)).cuda()
    out = ops.dequant_u4(torch.from_numpy(rhs).cuda(), st, zt, group)
    want = oracle.dequant_u4_ref(rhs, sc, zr, K, N, group, dt)
    assert np.array_equal(out.cpu().view(torch.int16).numpy().view(np.uint16), want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("wt", [False, True])
def test_dense_gemm_vs_torch(dev, dtype, wt):
    M, K, N = 200, 320, 136
    a = torch.randn(M, K, device=dev).to(dtype)
    w = torch.randn(N, K, device=dev).to(dtype) if wt else torch.randn(K, N, device=dev).to(dtype)
    out = ops.gemm_dense(a, w, w_transposed=wt)
    want = a.double() @ (w.double().T if wt else w.double())
    assert (torch.linalg.norm(out.double() - want) / torch.linalg.norm(want)).item() < 1e-2
    # matmul_* takes the library GEMM (hipBLASLt) at this size: GEMM tolerance;
    # with the w4a16_path = 1 knob the same MFMA core as ubridge_gemm_dense
    ref = ops.matmul(a, w, rhs_transpose=wt)
    assert ((ref.double() - out.double()).norm() / out.double().norm()).item() < 4e-3
    ops.tune_set("w4a16_path", 1)
    try:
        core = ops.matmul(a, w, rhs_transpose=wt)
    finally:
        ops.tune_set("w4a16_path", 0)
    assert torch.equal(core, out)


def test_batched_matmul_reference(dev):
    B, M, K, N = 3, 40, 128, 64
    a = torch.randn(B, M, K, device=dev).bfloat16()
    w = torch.randn(B, K, N, device=dev).bfloat16()
    out = ops.matmul(a, w)
    want = torch.bmm(a.double(), w.double())
    assert (torch.linalg.norm(out.double() - want) / torch.linalg.norm(want)).item() < 1e-2


def test_gemm_rejects_bad_shapes(dev):
    a = torch.zeros(4, 12, device=dev, dtype=torch.bfloat16)
    with pytest.raises(Exception):
        ops.w4a16_gemm(a, torch.zeros(1, 8, dtype=torch.int32, device=dev),
                       torch.zeros(1, 8, dtype=torch.bfloat16, device=dev),
                       torch.zeros(1, 1, dtype=torch.int32, device=dev), 128)


@pytest.mark.parametrize("sip", [(0, 0), (128, 128), (128, 256), (256, 256), (32, 64)])
def test_matmul_8bit_tile_from_launch_params(dev, sip):
    # the caller's order of the reference: get_gemm_launch_params, then
    # matmul_* with its sip_* fields.  Named tiles are honoured, anything else
    # falls back to the shape rule; every tile gives the oracle's result to
    # the GEMM tolerance, and the getter's own tile equals the default launch
    # bit for bit.
    M, K, N = 200, 512, 520
    g = np.random.default_rng(7)
    w = g.integers(-127, 128, (K, N)).astype(np.int8)
    sc = synth.f32_to_bf16_bits(g.uniform(0.002, 0.02, (1, N)).astype(np.float32))
    a = synth.bf16_activations(M, K, seed=8)
    at, wt, st = _bf(a), torch.from_numpy(w).cuda(), _bf(sc)
    out = torch.empty(1, M, N, dtype=torch.bfloat16, device=dev)
    args = [5, 1, M, K, N, 0, 0, 0, 0, 0, 1.0, 0.0, 0.0, sip[0], 64, sip[1], 1]
    _lib.lib.matmul_bf16_8bit(at.data_ptr(), wt.data_ptr(), out.data_ptr(), st.data_ptr(), None,
                              *args, -1, None)
    _lib.check()
    want = oracle.w8a16_gemm(a, w, sc, M, K, N, -1, 0)
    assert rel_err(oracle.bf16_to_f32(_np(out[0])), oracle.bf16_to_f32(want)) < 1e-2
    dflt = ops.matmul_quant(at, wt, st, bits=8)  # sip_* from the getter
    p = ops.get_gemm_launch_params(torch.bfloat16, "i8", 1, M, K, N, 0)
    if sip in ((0, 0), (p.sip_m, p.sip_n)):
        assert torch.equal(dflt.view(torch.int16), out[0].view(torch.int16))


# ---- reference-layout quantized GEMMs on the pipelined kernel (matmul_*_{4,8}bit)

def _t(bits, dtype):  # uint16 bits -> torch tensor of dtype on the GPU
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(dtype)


def _round_t(x32, dtype):  # f32 -> T bits (round to nearest even)
    if dtype == torch.bfloat16:
        return synth.f32_to_bf16_bits(x32.astype(np.float32))
    return x32.astype(np.float32).astype(np.float16).view(np.uint16)


def _to_f32(bits, dtype):
    if dtype == torch.bfloat16:
        return oracle.bf16_to_f32(bits)
    return bits.view(np.float16).astype(np.float32)


def _quant_case(bits, rhs_t, M, K, N, group, dtype, seed):
    """Random reference-layout weights + activations; returns the tensors
    and the exactly dequantized weight [K, N] (f32 image of T values)."""
    g = np.random.default_rng(seed)
    ng = 1 if group == -1 else K // group
    gs = K if group == -1 else group
    sc = _round_t(g.uniform(0.002, 0.02, (ng, N)), dtype)
    a = _round_t(g.standard_normal((M, K)), dtype)
    if bits == 8:
        w = g.integers(-128, 128, (N, K) if rhs_t else (K, N)).astype(np.int8)
        wk = (w.T if rhs_t else w).astype(np.float32)
        s_full = np.repeat(_to_f32(sc, dtype), gs, axis=0)
        wd = _to_f32(_round_t(wk * s_full, dtype), dtype)  # T(q s), q s exact in f32
        zt = None
    else:
        w = g.integers(0, 256, (K // 2, N)).astype(np.uint8)
        zr = _round_t(g.integers(0, 16, (ng, N)) + g.choice([0.0, 0.5, 0.3], (ng, N)), dtype)
        wdb = oracle.dequant_u4_ref(w, sc, zr, K // 2, N, gs,
                                    oracle.BF16 if dtype == torch.bfloat16 else oracle.F16)
        wd = _to_f32(wdb, dtype)
        zt = _t(zr, dtype)
    return _t(a, dtype), torch.from_numpy(w).cuda(), _t(sc, dtype), zt, \
        _to_f32(a, dtype), wd


def _exact_weight(bits, rhs_t, w, sc, zt, K, N, group, dtype):
    """The dequantized weight [K, N] in f64 without any rounding: (q - z) s
    (4-bit) or q s (int8)."""
    gs = K if group == -1 else group
    s = np.repeat(sc.float().cpu().numpy().astype(np.float64), gs, axis=0)
    wn = w.cpu().numpy()
    if bits == 8:
        return (wn.T if rhs_t else wn).astype(np.float64) * s
    q = np.empty((K, N), np.float64)
    q[0::2], q[1::2] = wn & 15, wn >> 4
    z = np.repeat(zt.float().cpu().numpy().astype(np.float64), gs, axis=0)
    return (q - z) * s


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bits,rhs_t", [(4, 0), (8, 0), (8, 1)])
@pytest.mark.parametrize("tile", [0, 1, 3])
@pytest.mark.parametrize("M,K,N,group", [(300, 1152, 520, 128), (77, 576, 264, 64),
                                         (256, 128, 512, -1), (40, 64, 8, 64),
                                         (40, 1024, 264, 128)])
def test_matmul_quant_pipelined(dev, dtype, bits, rhs_t, tile, M, K, N, group):
    # against an f64 product of the exactly dequantized weight: the bf16 / f16
    # outputs of an f32 accumulation agree to T rounding; K = 576 and 64 leave
    # no split-K variant, N = 8 and 264 cut the last column tile; 40 x 1024
    # runs the 64-row wave tiles with K also split over workgroups
    a, w, sc, zt, a32, wd = _quant_case(bits, rhs_t, M, K, N, group, dtype, M + K + bits)
    ops.tune_set("gemm_tile", tile)
    try:
        out = ops.matmul_quant(a, w, sc, zt, bits=bits, group_size=group,
                               rhs_transpose=bool(rhs_t))
    finally:
        ops.tune_set("gemm_tile", 0)
    want = a32.astype(np.float64) @ wd.astype(np.float64)
    got = out.float().cpu().numpy().astype(np.float64)
    assert rel_err(got, want) < 1e-2
    want_t = _to_f32(_round_t(want, dtype), dtype)
    assert np.mean(got == want_t) > 0.9


@pytest.mark.parametrize("bits,rhs_t", [(4, 0), (8, 0), (8, 1)])
def test_matmul_quant_pipelined_matches_core(dev, bits, rhs_t):
    # the pipelined kernel and the generic MFMA core (w4a16_path = 1) compute
    # the same dequantized products; f32 sums in different orders, so equal
    # to T rounding
    M, K, N, group = 520, 1024, 768, 128
    a, w, sc, zt, _, _ = _quant_case(bits, rhs_t, M, K, N, group, torch.bfloat16, 9)
    fast = ops.matmul_quant(a, w, sc, zt, bits=bits, group_size=group, rhs_transpose=bool(rhs_t))
    ops.tune_set("w4a16_path", 1)
    try:
        core = ops.matmul_quant(a, w, sc, zt, bits=bits, group_size=group,
                                rhs_transpose=bool(rhs_t))
    finally:
        ops.tune_set("w4a16_path", 0)
    d = (fast.double() - core.double()).norm() / core.double().norm()
    assert d.item() < 4e-3
    assert (fast == core).float().mean().item() > 0.9


@pytest.mark.parametrize("bits,rhs_t", [(4, 0), (8, 1)])
@pytest.mark.parametrize("M", [512, 2048])
def test_matmul_quant_cfg3_shape(dev, bits, rhs_t, M):
    # configs[2]'s shape (K = 4096, N = 14336, g = 128) in the reference
    # layouts, batched as B = 2 x M/2 (the batches fold into M), checked per
    # 256-row band against an f64 GPU product of the exact dequantized weight
    K, N, group = 4096, 14336, 128
    a, w, sc, zt, _, wd = _quant_case(bits, rhs_t, M, K, N, group, torch.bfloat16, 3)
    out = ops.matmul_quant(a.view(2, M // 2, K), w, sc, zt, bits=bits, group_size=group,
                           rhs_transpose=bool(rhs_t)).view(M, N)
    want = a.double() @ torch.from_numpy(wd).cuda().double()
    band = [(torch.linalg.norm(out[i:i + 256].double() - want[i:i + 256]) /
             torch.linalg.norm(want[i:i + 256])).item() for i in range(0, M, 256)]
    assert max(band) < 1e-2, band


def test_launch_params_name_the_pipelined_tile(dev):
    # quantized weights: the getter describes the pipelined kernel's tile
    p = ops.get_gemm_launch_params(torch.bfloat16, "i4", 1, 512, 4096, 14336, 0)
    assert (p.sip_m, p.sip_k, p.sip_n) == (128, 64, 256)
    p = ops.get_gemm_launch_params(torch.bfloat16, "i8", 1, 2048, 4096, 14336, 1)
    assert (p.sip_m, p.sip_k, p.sip_n) == (256, 64, 256)
    p = ops.get_gemm_launch_params(torch.bfloat16, "i4", 1, 64, 4096, 14336, 0)
    assert (p.sip_m, p.sip_k, p.sip_n) == (64, 64, 256)  # 64-row tiles up to 64 rows


# ---- decode-shape GEMV (M <= 16) of the k-major quantized layouts

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bits,rhs_t", [(4, 0), (8, 0), (8, 1)])
@pytest.mark.parametrize("M,K,N,group", [(1, 4096, 14336, 128), (3, 1024, 264, 64),
                                         (16, 512, 520, -1), (7, 64, 8, 32), (2, 14336, 4096, 128),
                                         (2, 1152, 200, 96), (9, 4096, 1000, 64)])
def test_matmul_quant_decode_gemv(dev, dtype, bits, rhs_t, M, K, N, group):
    # up to 16 tokens take the decode GEMV, which applies scale and zero
    # point once per group to the f32 MFMA sum (the weight unrounded): within
    # the GEMM tolerance of the f64 product of the T-rounded dequantized
    # weight (the contract), equal to T rounding of the f64 product of the
    # unrounded weight, and within tolerance of the pipelined GEMM (knob
    # w4a16_path = 2)
    # int8 [N, K] reads k in pairs of steps: groups of 32 or 96 take the GEMM
    # path instead (the decode GEMV declines them), covered all the same
    a, w, sc, zt, a32, wd = _quant_case(bits, rhs_t, M, K, N, group, dtype, M * 7 + K + bits)
    out = ops.matmul_quant(a, w, sc, zt, bits=bits, group_size=group, rhs_transpose=bool(rhs_t))
    got = out.float().cpu().numpy().astype(np.float64)
    assert rel_err(got, a32.astype(np.float64) @ wd.astype(np.float64)) < 1e-2
    wx = _exact_weight(bits, rhs_t, w, sc, zt, K, N, group, dtype)
    want_t = _to_f32(_round_t(a32.astype(np.float64) @ wx, dtype), dtype)
    if not (bits == 8 and rhs_t and group % 64):
        assert np.mean(got == want_t) > 0.85
    ops.tune_set("w4a16_path", 2)
    try:
        gemm = ops.matmul_quant(a, w, sc, zt, bits=bits, group_size=group,
                                rhs_transpose=bool(rhs_t))
    finally:
        ops.tune_set("w4a16_path", 0)
    d = (out.double() - gemm.double()).norm() / gemm.double().norm()
    assert d.item() < 4e-3


@pytest.mark.parametrize("M,K,N,group", [(1, 4096, 14336, 128), (16, 4096, 4096, 128),
                                         (5, 256, 72, 32), (1, 4096, 8192, 128),
                                         (3, 2048, 10248, 64), (16, 1024, 14336, 128),
                                         (2, 4096, 16384, 128)])
def test_w4a16_decode_gemv(dev, M, K, N, group):
    # GPTQ decode GEMV, narrow and wide grids (10248: a partial last column
    # block)
    qw, sc, qz = synth.make_gptq_w4(K, N, group, seed=M + N)
    a = synth.bf16_activations(M, K, seed=K)
    out = ops.w4a16_gemm(_bf(a), torch.from_numpy(qw).cuda(), _bf(sc), torch.from_numpy(qz).cuda(),
                         group)
    wd = torch.from_numpy(oracle.bf16_to_f32(oracle.w4a16_dequant(qw, sc, qz, K, N, group))).cuda()
    want = _bf(a).double() @ wd.double()
    err = (torch.linalg.norm(out.double() - want) / torch.linalg.norm(want)).item()
    assert err < 1e-2, err
    # the GEMV scales the unrounded weight: T rounding of its f64 product
    q = np.empty((K, N), np.float64)
    for i in range(8):
        q[i::8] = (qw >> (4 * i)) & 15
    z = np.empty((K // group, N), np.float64)
    for i in range(8):
        z[:, i::8] = (qz >> (4 * i)) & 15
    s = oracle.bf16_to_f32(sc).astype(np.float64)
    wx = (q - np.repeat(z, group, 0)) * np.repeat(s, group, 0)
    exact = _bf(a).double() @ torch.from_numpy(wx).cuda()
    assert (out == exact.bfloat16()).float().mean().item() > 0.85


def test_decode_gemv_ksplit_graph_capture(dev):
    # a narrow matrix takes the K split through a stream workspace: captured on
    # a fresh stream (no workspace yet) the single-launch form is recorded,
    # captured after an eager call the split form; every replay of both graphs
    # equals the eager result (f32 sums in the same fixed orders)
    M, K, N, group = 2, 14336, 4096, 128
    qw, sc, qz = synth.make_gptq_w4(K, N, group, seed=11)
    a = _bf(synth.bf16_activations(M, K, seed=12))
    qw, qz, sct = torch.from_numpy(qw).cuda(), torch.from_numpy(qz).cuda(), _bf(sc)
    for warm in (False, True):
        s = torch.cuda.Stream()
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        if warm:
            with torch.cuda.stream(s):
                ops.w4a16_gemm(a, qw, sct, qz, group, out=out, stream=s)
            torch.cuda.synchronize()
        eager = out.clone()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            ops.w4a16_gemm(a, qw, sct, qz, group, out=out, stream=s)
        for _ in range(3):
            out.zero_()
            g.replay()
            torch.cuda.synchronize()
            if warm:
                assert torch.equal(out, eager)
            else:
                d = (out.double() - eager.double()).norm() / eager.double().norm()
                assert d.item() < 4e-3 if eager.abs().sum() > 0 else True
        if not warm:  # the eager result of the split form vs the recorded one
            with torch.cuda.stream(s):
                ops.w4a16_gemm(a, qw, sct, qz, group, out=eager, stream=s)
            torch.cuda.synchronize()
            d = (out.double() - eager.double()).norm() / eager.double().norm()
            assert d.item() < 4e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("wt", [False, True])
@pytest.mark.parametrize("B,M,K,N", [(1, 1, 4096, 1024), (1, 5, 1024, 264), (1, 16, 2048, 4096),
                                     (2, 3, 512, 136)])
def test_dense_matmul_decode_gemv(dev, dtype, wt, B, M, K, N):
    # matmul_{bf16,f16} at up to 16 tokens (x batch, one broadcast weight)
    # takes the decode GEMV: against the f64 product and the MFMA core (knob 1)
    g = torch.Generator(device=dev).manual_seed(M * N + K)
    a = torch.randn(B, M, K, device=dev, generator=g).to(dtype)
    w = (torch.randn(N, K, device=dev, generator=g) if wt else
         torch.randn(K, N, device=dev, generator=g)).to(dtype)
    out = ops.matmul(a, w, rhs_transpose=wt)
    want = a.double() @ (w.double().T if wt else w.double())
    assert (torch.linalg.norm(out.double() - want) / torch.linalg.norm(want)).item() < 1e-2
    ops.tune_set("w4a16_path", 1)
    try:
        core = ops.matmul(a, w, rhs_transpose=wt)
    finally:
        ops.tune_set("w4a16_path", 0)
    d = (out.double() - core.double()).norm() / core.double().norm()
    assert d.item() < 4e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("wt", [False, True])
@pytest.mark.parametrize("B,M,K,N,bcast", [(1, 200, 320, 136, True), (3, 40, 128, 64, False),
                                           (2, 130, 512, 264, True), (1, 17, 4096, 1024, True)])
def test_dense_matmul_library_gemm(dev, dtype, wt, B, M, K, N, bcast):
    # beyond 16 tokens matmul_{bf16,f16} is a hipBLASLt GEMM (per-batch or
    # broadcast weights): against the f64 product and the MFMA core
    g = torch.Generator(device=dev).manual_seed(M + N + K + B)
    a = torch.randn(B, M, K, device=dev, generator=g).to(dtype)
    shape = (N, K) if wt else (K, N)
    w = torch.randn(*((shape) if bcast else (B, *shape)), device=dev, generator=g).to(dtype)
    out = ops.matmul(a, w, rhs_transpose=wt)
    wd = w.double().transpose(-1, -2) if wt else w.double()
    want = a.double() @ wd
    assert (torch.linalg.norm(out.double() - want) / torch.linalg.norm(want)).item() < 1e-2
    ops.tune_set("w4a16_path", 1)
    try:
        core = ops.matmul(a, w, rhs_transpose=wt)
    finally:
        ops.tune_set("w4a16_path", 0)
    assert ((out.double() - core.double()).norm() / core.double().norm()).item() < 4e-3


def _slab_vs_core(run):
    fast = run()
    ops.tune_set("w4a16_path", 1)
    try:
        core = run()
    finally:
        ops.tune_set("w4a16_path", 0)
    torch.cuda.synchronize()
    d = (fast.double() - core.double()).norm() / core.double().norm()
    assert d.item() < 4e-3, d.item()
    # both round the same f32 products of the same T weights: most outputs equal
    assert (fast == core).float().mean().item() > 0.9
    return fast


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bits,rhs_t", [(4, 0), (8, 0), (8, 1)])
@pytest.mark.parametrize("M,K,N,group", [(700, 1024, 776, 128), (1536, 1024, 776, 128),
                                         (2100, 8192, 16400, 64)])
def test_matmul_quant_slab_route(dev, dtype, bits, rhs_t, M, K, N, group):
    # beyond 1024 tokens (uint8 4-bit: from 640; M = 700 keeps int8 on the
    # pipelined kernel) the weight is dequantized into T slabs (at most 256 MB:
    # K = 8192, N = 16400 takes 16384 columns and a 16-column tail) and each
    # slab goes through hipBLASLt; against the MFMA core's fused dequantization
    a, w, sc, zt, _, _ = _quant_case(bits, rhs_t, M, K, N, group, dtype, M + bits)
    _slab_vs_core(lambda: ops.matmul_quant(a, w, sc, zt, bits=bits, group_size=group,
                                           rhs_transpose=bool(rhs_t)))


@pytest.mark.parametrize("M,K,N,group", [(1100, 4096, 14336, 128), (2048, 1152, 520, 96),
                                         (1600, 8192, 16400, 128)])
def test_w4a16_slab_route(dev, M, K, N, group):
    qw, sc, qz = synth.make_gptq_w4(K, N, group, seed=M)
    a = synth.bf16_activations(M, K, seed=K)
    args = (_bf(a), torch.from_numpy(qw).cuda(), _bf(sc), torch.from_numpy(qz).cuda(), group)
    _slab_vs_core(lambda: ops.w4a16_gemm(*args))


def test_slab_route_graph_capture(dev):
    # the slab route needs scratch and hipBLASLt plans; both are obtained
    # outside the capture when first needed inside one, so a graph captured on
    # a fresh stream records the same dequantization + hipBLASLt launches as
    # one captured after an eager call, and every replay (the scratch
    # rewritten each time) equals the eager result bit for bit
    M, K, N, group = 1536, 1024, 776, 128
    qw, sc, qz = synth.make_gptq_w4(K, N, group, seed=21)
    a = _bf(synth.bf16_activations(M, K, seed=22))
    qw, qz, sct = torch.from_numpy(qw).cuda(), torch.from_numpy(qz).cuda(), _bf(sc)
    ref = ops.w4a16_gemm(a, qw, sct, qz, group)  # default stream: the slab route
    torch.cuda.synchronize()
    for warm in (False, True):
        s = torch.cuda.Stream()
        out = torch.zeros(M, N, dtype=torch.bfloat16, device=dev)
        if warm:
            with torch.cuda.stream(s):
                ops.w4a16_gemm(a, qw, sct, qz, group, out=out, stream=s)
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            ops.w4a16_gemm(a, qw, sct, qz, group, out=out, stream=s)
        for _ in range(3):
            out.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
            _ = ops.w4a16_gemm(a, qw, sct, qz, group)  # eager work between replays


@pytest.mark.parametrize("M", [17, 64, 200])
def test_pipelined_k_split_over_workgroups(dev, M):
    # grids under half the CUs split K over 2-8 workgroups per tile (f32
    # partials summed in a fixed order); knob w4a16_path = 7 runs them
    # unsplit: the same products in another f32 order
    K, N, group = 4096, 1024, 128
    qw, sc, qz = synth.make_gptq_w4(K, N, group, seed=M)
    a = _bf(synth.bf16_activations(M, K, seed=M + 1))
    args = (a, torch.from_numpy(qw).cuda(), _bf(sc), torch.from_numpy(qz).cuda(), group)
    a8, w8, sc8, _, _, _ = _quant_case(8, 1, M, K, N, group, torch.bfloat16, M)
    a4, w4, sc4, zt4, _, _ = _quant_case(4, 0, M, K, N, group, torch.float16, M + 2)  # f16 sums
    runs = [lambda: ops.w4a16_gemm(*args),
            lambda: ops.matmul_quant(a8, w8, sc8, None, bits=8, group_size=group, rhs_transpose=True),
            lambda: ops.matmul_quant(a4, w4, sc4, zt4, bits=4, group_size=group)]
    for run in runs:
        split = run()
        ops.tune_set("w4a16_path", 7)
        try:
            whole = run()
        finally:
            ops.tune_set("w4a16_path", 0)
        d = (split.double() - whole.double()).norm() / whole.double().norm()
        assert d.item() < 4e-3
        assert (split == whole).float().mean().item() > 0.9


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", [128, 40])
def test_pipelined_dequant_bit_exact(dev, dtype, M):
    # one-hot activation rows (row i picks k = i): every output is one
    # dequantized weight times 1, exact whatever the summation order, so the
    # pipelined kernel's B operands (and its 64-row tiles / K split at 40
    # rows) are pinned bit for bit against the dequantizers
    K, N, group = 128, 264, 64
    eye = torch.zeros(M, K, dtype=dtype, device=dev)
    eye[torch.arange(M), torch.arange(M)] = 1
    # uint8 4-bit: dequant_{bf16,f16}
    a, w, sc, zt, _, _ = _quant_case(4, 0, M, K, N, group, dtype, 5)
    got = ops.matmul_quant(eye, w, sc, zt, bits=4, group_size=group)
    want = ops.dequant_u4(w, sc, zt, group_size=group).view(K, N)[:M]
    assert torch.equal(got.view(torch.int16), want.contiguous().view(torch.int16))
    # int8 [N, K]: T(q s)
    _, w8, sc8, _, _, _ = _quant_case(8, 1, M, K, N, group, dtype, 6)
    got = ops.matmul_quant(eye, w8, sc8, None, bits=8, group_size=group, rhs_transpose=True)
    s_full = sc8.float().repeat_interleave(group, 0)
    want = (w8.float().t() * s_full).to(dtype)[:M]
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    if dtype == torch.bfloat16:  # GPTQ against the oracle's bit-exact dequant
        qw, scg, qz = synth.make_gptq_w4(K, N, group, seed=7)
        got = ops.w4a16_gemm(eye, torch.from_numpy(qw).cuda(), _bf(scg), torch.from_numpy(qz).cuda(),
                             group)
        want = oracle.w4a16_dequant(qw, scg, qz, K, N, group)[:M]
        assert np.array_equal(_np(got), want)


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0, ops.Q4_K])
def test_qmatmul_pipelined_dequant_bit_exact(dev, qt):
    # the same with QMatMul's GGUF producers: x one-hot (bf16), y f32 =
    # dequantize_block_*_bf16 exactly (transposed)
    K, N, M = 256, 264, 256
    w = torch.from_numpy(synth.make_weight_soa(qt, N, K, seed=8)).to(dev)
    x = torch.zeros(M, K, dtype=torch.bfloat16, device=dev)
    x[torch.arange(M), torch.arange(M)] = 1
    ops.tune_set("w4a16_path", 4)
    try:
        y = ops.QMatMul(qt, w, N, K)(x)
    finally:
        ops.tune_set("w4a16_path", 0)
    wd = ops.dequantize_block(qt, w, N * K, torch.bfloat16).view(N, K).float()
    assert torch.equal(y, wd.t().contiguous())


def test_k_split_graph_capture(dev):
    # the K split needs scratch: captured on a fresh stream (the pool grown
    # outside the capture) or after an eager call, the graph records the
    # split kernel and the partial-sum launch, and every replay equals the
    # eager result bit for bit
    M, K, N, group = 64, 4096, 2048, 128
    qw, sc, qz = synth.make_gptq_w4(K, N, group, seed=31)
    a = _bf(synth.bf16_activations(M, K, seed=32))
    qw, qz, sct = torch.from_numpy(qw).cuda(), torch.from_numpy(qz).cuda(), _bf(sc)
    ref = ops.w4a16_gemm(a, qw, sct, qz, group)
    torch.cuda.synchronize()
    for warm in (False, True):
        s = torch.cuda.Stream()
        out = torch.zeros(M, N, dtype=torch.bfloat16, device=dev)
        if warm:
            with torch.cuda.stream(s):
                ops.w4a16_gemm(a, qw, sct, qz, group, out=out, stream=s)
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            ops.w4a16_gemm(a, qw, sct, qz, group, out=out, stream=s)
        for _ in range(3):
            out.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
            _ = ops.w4a16_gemm(a, qw, sct, qz, group)  # eager work between replays


@pytest.mark.parametrize("M", [64, 512])
def test_w4a16_misaligned_a(dev, M):
    # A 2 bytes past 16-byte alignment: copied once into call scratch, then
    # the same route as the aligned call (bit-identical); also for the
    # reference-layout matmul_bf16_8bit
    K, N, group = 1024, 776, 128
    qw, sc, qz = synth.make_gptq_w4(K, N, group, seed=M)
    a = _bf(synth.bf16_activations(M, K, seed=M + 1))
    buf = torch.zeros(M * K + 1, dtype=torch.bfloat16, device=dev)
    buf[1:] = a.reshape(-1)
    am = buf[1:].view(M, K)
    assert am.data_ptr() % 16 == 2
    args = (torch.from_numpy(qw).cuda(), _bf(sc), torch.from_numpy(qz).cuda(), group)
    print(f"misaligned w4a16 M={M}", flush=True)
    assert torch.equal(ops.w4a16_gemm(am, *args), ops.w4a16_gemm(a, *args))
    w8 = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev)
    s8 = (torch.rand(1, N, device=dev) * 0.01 + 0.001).to(torch.bfloat16)
    r1 = ops.matmul_quant(am, w8, s8, bits=8, rhs_transpose=True)
    r2 = ops.matmul_quant(a, w8, s8, bits=8, rhs_transpose=True)
    assert torch.equal(r1, r2)
