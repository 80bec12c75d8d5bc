"""Pin the CPU oracle (oracle/ubridge_oracle.c) before trusting it.

Each check is chosen so that a plausible mistake in the oracle -- a dropped
term, a wrong sign, a swapped nibble, an off-by-one scale index -- fails:
  * exhaustive / library comparisons for the scalar conversions;
  * bit-exact comparison with the independent numpy restatement in
    tests/golden/make_golden.py (golden.npz);
  * closed forms: exactly representable activations make Candle's activation
    quantization lossless, so QMatMul must equal the f64 dense dot;
  * invariants (round trips, permutation / padding rules) and brute force.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import rel_err
from ubridge_amd import synth


# ------------------------------------------------------------ conversions
def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32_scalar(int(b)) for b in bits[::7]], np.float32)
    w = want[::7]
    ok = (got == w) | (np.isnan(got) & np.isnan(w))
    assert ok.all()


def test_f32_to_f16_rne():
    g = np.random.default_rng(1)
    vals = np.concatenate([g.standard_normal(3000) * 10 ** g.uniform(-9, 5, 3000),
                           [65504, 65519.99, 65520, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 0.0,
                            -0.0, 1e-30, 1e30]]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)

    got = np.array([oracle.f32_to_f16_scalar(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


def test_bf16_matches_torch():
    g = np.random.default_rng(2)
    x = (g.standard_normal(20000) * 10 ** g.uniform(-30, 30, 20000)).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.f32_to_bf16(x), want)
    assert np.array_equal(oracle.bf16_to_f32(want), torch.from_numpy(want.view(np.int16)).view(
        torch.bfloat16).float().numpy())


def test_e4m3_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = np.array([oracle.e4m3_to_f32(c) for c in codes], np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    m = ~np.isnan(want)
    assert np.array_equal(got[m], want[m])
    g = np.random.default_rng(3)
    x = np.clip(g.standard_normal(5000) * 10 ** g.uniform(-4, 2.5, 5000), -448, 448).astype(np.float32)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = np.array([oracle.f32_to_e4m3(v) for v in x], np.uint8)
    assert np.array_equal(got, want)


# --------------------------------------------------------------- dequant
@pytest.mark.parametrize("name,qt,bk", [("q8_0", oracle.Q8_0, 32), ("q4_0", oracle.Q4_0, 32),
                                        ("q4_k", oracle.Q4_K, 256)])
@pytest.mark.parametrize("dt,suffix", [(oracle.F32, "f32"), (oracle.F16, "f16"),
                                       (oracle.BF16, "bf16")])
def test_dequant_matches_golden(golden, name, qt, bk, dt, suffix):
    soa = golden[f"{name}_soa"]
    want = golden[f"{name}_{suffix}"]
    got = oracle.dequant(qt, soa, want.size, dt)
    if dt == oracle.F32:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    else:
        assert np.array_equal(got, want)


def test_dequant_closed_forms():
    # Q8_0 with d = 1: output is the code itself
    nb = 4
    q = np.arange(-64, 64, dtype=np.int8)
    soa = np.concatenate([np.full(nb, 0x3C00, np.uint16).view(np.uint8), q.view(np.uint8)])
    assert np.array_equal(oracle.dequant(oracle.Q8_0, soa, 128, oracle.F32), q.astype(np.float32))
    # Q4_0: code 8 -> 0 for any d; nibble order lo = j, hi = j + 16
    qs = np.zeros(16, np.uint8)
    qs[3] = 0x8F  # element 3 -> 15-8 = 7, element 19 -> 8-8 = 0
    soa = np.concatenate([np.array([0x4000], np.uint16).view(np.uint8), qs])  # d = 2
    out = oracle.dequant(oracle.Q4_0, soa, 32, oracle.F32)
    want = np.full(32, -16.0, np.float32)
    want[3], want[19] = 14.0, 0.0
    assert np.array_equal(out, want)
    # Q4_K: d=1, dmin=1, sub-block scales = s+1, mins = s: y = (s+1)*q - s
    hdr = np.zeros(16, np.uint8)
    hdr[0:2] = np.array([0x3C00], np.uint16).view(np.uint8)
    hdr[2:4] = np.array([0x3C00], np.uint16).view(np.uint8)
    sc = np.arange(1, 9)
    mn = np.arange(0, 8)
    b = hdr[4:16]
    b[0:4] = sc[0:4] | ((sc[4:8] >> 4) << 6)
    b[4:8] = mn[0:4] | ((mn[4:8] >> 4) << 6)
    b[8:12] = (sc[4:8] & 15) | ((mn[4:8] & 15) << 4)
    codes = np.arange(256) % 16
    qs = np.zeros(128, np.uint8)
    for j in range(4):
        qs[32 * j:32 * j + 32] = codes[64 * j:64 * j + 32] | (codes[64 * j + 32:64 * j + 64] << 4)
    out = oracle.dequant(oracle.Q4_K, np.concatenate([hdr, qs]), 256, oracle.F32)
    sub = np.arange(256) // 32
    assert np.array_equal(out, ((sub + 1) * codes - sub).astype(np.float32))


@pytest.mark.parametrize("qt", [oracle.Q4_0, oracle.Q8_0, oracle.Q4_K])
def test_aos_soa_roundtrip(qt):
    w = synth.make_weight_soa(qt, 8, 512, seed=3)
    nb = 8 * 512 // (256 if qt == oracle.Q4_K else 32)
    aos = oracle.soa_to_aos(qt, w, nb)
    hb = 16 if qt == oracle.Q4_K else 2
    bb = {oracle.Q4_0: 16, oracle.Q8_0: 32, oracle.Q4_K: 128}[qt]
    assert np.array_equal(aos.reshape(nb, hb + bb)[:, :hb].ravel(), w[: nb * hb])
    assert np.array_equal(oracle.aos_to_soa(qt, aos, nb), w)


# ------------------------------------------------------ activation quant
def test_quantize_q8_0_golden(golden):
    soa = oracle.quantize_q8_0(golden["act_x"])
    nb = golden["act_x"].size // 32
    assert np.array_equal(soa[: 2 * nb].view(np.uint16), golden["q8_0_d"])
    assert np.array_equal(soa[2 * nb:].view(np.int8), golden["q8_0_q"])


def test_quantize_q8_k_golden(golden):
    d, q, bs = oracle.quantize_q8_k(golden["act_x"])
    assert np.array_equal(d.view(np.uint32), golden["q8_k_d"].view(np.uint32))
    assert np.array_equal(q, golden["q8_k_q"])
    assert np.array_equal(bs, golden["q8_k_bs"])


def test_quantize_invariants():
    x = synth.make_activations(4, 1024, seed=5).ravel()
    soa = oracle.quantize_q8_0(x)
    nb = x.size // 32
    d = soa[: 2 * nb].view(np.float16).astype(np.float32)
    q = soa[2 * nb:].view(np.int8).reshape(nb, 32)
    assert np.abs(q).max() <= 127
    assert (np.abs(q).max(axis=1) == 127).all()  # amax maps to 127
    err = np.abs(q * d[:, None] - x.reshape(nb, 32))
    # codes use the f32 d, dequant the fp16-rounded d: 127 * 2^-11 * d on top of d/2
    assert (err <= d[:, None] * (0.5 + 127 * 2.0**-11) * 1.001 + 1e-7).all()
    dk, qk, bsk = oracle.quantize_q8_k(x)
    assert (qk.reshape(-1, 256).min(axis=1) >= -128).all() and qk.max() <= 127
    assert np.array_equal(bsk, qk.reshape(-1, 16, 16).astype(np.int32).sum(axis=2).ravel())


# ---------------------------------------------------------------- qmatmul
@pytest.mark.parametrize("name,qt", [("mm_q4_0", oracle.Q4_0), ("mm_q8_0", oracle.Q8_0),
                                     ("mm_q4_k", oracle.Q4_K)])
def test_qmatmul_golden(golden, name, qt):
    N, K = golden[f"{name}_shape"]
    y = oracle.qmatmul(qt, golden[f"{name}_w"], golden[f"{name}_x"], int(N), int(K))
    assert rel_err(y, golden[f"{name}_y"]) < 2e-6


def _exact_activations(M, K, blk, seed):
    """Integer activations whose Q8_0 (amax 127) / Q8_K (max -128) quantization
    is lossless, so Candle's method must equal the exact dense dot."""
    g = np.random.default_rng(seed)
    x = g.integers(-120, 121, (M, K)).astype(np.float32)
    if blk == 32:
        x.reshape(M, -1, 32)[:, :, 5] = 127.0
    else:
        x.reshape(M, -1, 256)[:, :, 17] = -128.0
    return x


@pytest.mark.parametrize("qt", [oracle.Q4_0, oracle.Q8_0, oracle.Q4_K])
def test_qmatmul_exact_activations(qt):
    N, K, M = 40, 1024, 3
    w = synth.make_weight_soa(qt, N, K, seed=11)
    blk = 256 if qt == oracle.Q4_K else 32
    x = _exact_activations(M, K, blk, 12)
    y = oracle.qmatmul(qt, w, x, N, K)
    wd = oracle.dequant(qt, w, N * K, oracle.F32).reshape(N, K).astype(np.float64)
    want = x.astype(np.float64) @ wd.T
    assert rel_err(y, want) < 1e-6
    assert np.abs(y - want).max() <= 1e-5 * np.abs(want).max()


@pytest.mark.parametrize("qt", [oracle.Q4_0, oracle.Q8_0, oracle.Q4_K])
def test_qmatmul_quantization_bound(qt):
    N, K = 64, 4096
    w = synth.make_weight_soa(qt, N, K, seed=21)
    x = synth.make_activations(2, K, seed=22)
    y = oracle.qmatmul(qt, w, x, N, K, nthreads=4)
    wd = oracle.dequant(qt, w, N * K, oracle.F32).reshape(N, K).astype(np.float64)
    err = rel_err(y, x.astype(np.float64) @ wd.T)
    assert 1e-5 < err < 1e-2  # activation quantization is visible but bounded


def test_qmatmul_threads_agree():
    w = synth.make_weight_soa(oracle.Q4_K, 96, 512, seed=2)
    x = synth.make_activations(2, 512, seed=3)
    assert np.array_equal(oracle.qmatmul(oracle.Q4_K, w, x, 96, 512, 1),
                          oracle.qmatmul(oracle.Q4_K, w, x, 96, 512, 5))


# ------------------------------------------------------------ MoE routing
def test_topk_softmax_golden(golden):
    w, idx = oracle.topk_softmax(golden["topk_logits"], 4, True, oracle.F32)
    assert np.array_equal(idx, golden["topk_idx"])
    assert np.abs(w - golden["topk_w"]).max() < 1e-6
    w2, idx2 = oracle.topk_softmax(golden["topk_logits"], 4, False, oracle.F32)
    assert np.array_equal(idx2, golden["topk_idx_nonorm"])
    assert np.abs(w2 - golden["topk_w_nonorm"]).max() < 1e-6


def test_topk_softmax_ties_lowest_index():
    logits = np.zeros((2, 8), np.float32)
    logits[1, [2, 5, 6]] = 1.0
    w, idx = oracle.topk_softmax(logits, 3, False, oracle.F32)
    assert idx[0].tolist() == [0, 1, 2]
    assert idx[1].tolist() == [2, 5, 6]
    assert np.allclose(w[0], 1 / 8)


def test_moe_align_golden(golden):
    s, e, n = oracle.moe_align_block_size(golden["align_ids"], 8, 4)
    assert np.array_equal(s, golden["align_sorted"])
    assert np.array_equal(e, golden["align_experts"])
    assert n[0] == golden["align_ntpp"][0]


@pytest.mark.parametrize("T,k,E,bs", [(256, 8, 128, 16), (7, 2, 5, 4), (1, 1, 3, 8)])
def test_moe_align_invariants(T, k, E, bs):
    ids = np.random.default_rng(T).integers(0, E, (T, k)).astype(np.int32)
    s, e, n = oracle.moe_align_block_size(ids, E, bs)
    ntpp = int(n[0])
    assert ntpp % bs == 0
    valid = s[:ntpp][s[:ntpp] < T * k]
    assert np.array_equal(np.sort(valid), np.arange(T * k))  # every slot exactly once
    assert (s[ntpp:] == T * k).all()
    for b in range(ntpp // bs):
        blk = s[b * bs:(b + 1) * bs]
        real = blk[blk < T * k]
        assert (ids.ravel()[real] == e[b]).all()  # single-expert blocks
        assert np.all(np.diff(real) > 0)  # ascending slot order
    assert (e[ntpp // bs:] == 0).all()


def test_moe_align_expert_map_and_real_tokens():
    ids = np.array([[0, 1], [1, 2], [2, 2]], np.int32)
    emap = np.array([-1, 0, 1], np.int32)
    s, e, n = oracle.moe_align_block_size(ids, 3, 2, real_token_num=2, expert_map=emap)
    # only slots 0..3 count: expert 0 {0}, expert 1 {1,2}, expert 2 {3}
    assert n[0] == 6
    assert s[:6].tolist() == [0, 6, 1, 2, 3, 6]
    assert e[:3].tolist() == [-1, 0, 1]
    with pytest.raises(ValueError):
        oracle.moe_align_block_size(np.array([[3]], np.int32), 3, 2)


# ------------------------------------------------ GEMM / MoE oracles (brute force)
def _bf(x):
    return synth.f32_to_bf16_bits(np.asarray(x, np.float32))


def test_w8a16_oracle_brute_force():
    g = np.random.default_rng(1)
    M, K, N, group = 5, 64, 12, 16
    a = _bf(g.standard_normal((M, K)))
    w = g.integers(-127, 128, (K, N)).astype(np.int8)
    sc = _bf(g.uniform(0.002, 0.02, (K // group, N)))
    out = oracle.w8a16_gemm(a, w, sc, M, K, N, group, 0)
    wd = np.array([[synth.bf16_bits_to_f32(_bf(w[k, n] * synth.bf16_bits_to_f32(sc[k // group, n])))
                    for n in range(N)] for k in range(K)], np.float64).reshape(K, N)
    want = synth.bf16_bits_to_f32(a).astype(np.float64) @ wd
    assert np.array_equal(out, _bf(want.astype(np.float32)))
    out_t = oracle.w8a16_gemm(a, np.ascontiguousarray(w.T), sc, M, K, N, group, 1)
    assert np.array_equal(out_t, out)
    # group <= 0 means one group over all of K
    sc1 = _bf(g.uniform(0.002, 0.02, (1, N)))
    o1 = oracle.w8a16_gemm(a, w, sc1, M, K, N, -1, 0)
    o2 = oracle.w8a16_gemm(a, w, np.repeat(sc1, K, axis=0), M, K, N, 1, 0)
    assert np.array_equal(o1, o2)


def test_w4a16_oracle_brute_force():
    g = np.random.default_rng(2)
    K, N, group = 32, 16, 16
    qw, sc, qz = synth.make_gptq_w4(K, N, group, seed=9)
    wd = oracle.w4a16_dequant(qw, sc, qz, K, N, group)
    u = qw.view(np.uint32)
    uz = qz.view(np.uint32)
    for k in range(K):
        for n in range(N):
            q = (int(u[k // 8, n]) >> (4 * (k % 8))) & 15
            z = (int(uz[k // group, n // 8]) >> (4 * (n % 8))) & 15
            want = _bf(np.float32((q - z)) * synth.bf16_bits_to_f32(sc[k // group, n]))
            assert wd[k, n] == want
    a = _bf(g.standard_normal((3, K)))
    out = oracle.w4a16_gemm(a, qw, sc, qz, 3, K, N, group)
    ref = synth.bf16_bits_to_f32(a).astype(np.float64) @ synth.bf16_bits_to_f32(wd).astype(np.float64)
    assert np.array_equal(out, _bf(ref.astype(np.float32)))


def test_dequant_u4_ref_closed_form():
    rhs = np.array([[0x21, 0xF0]], np.uint8)  # 1 packed row -> rows 0 (low), 1 (high)
    sc = _bf([[0.5, 2.0]])
    zr = _bf([[1.0, 0.0]])
    out = synth.bf16_bits_to_f32(oracle.dequant_u4_ref(rhs, sc, zr, 1, 2, 2, oracle.BF16))
    assert out.tolist() == [[(1 - 1) * 0.5, 0.0], [(2 - 1) * 0.5, 15 * 2.0]]


def test_fp8_oracle():
    g = np.random.default_rng(3)
    x = (g.standard_normal((6, 40)) * 3).astype(np.float32)
    q, s = oracle.fp8_quantize_rows(x)
    dec = np.vectorize(oracle.e4m3_to_f32)(q)
    assert np.allclose(s, np.abs(x).max(axis=1) / 448, rtol=1e-7)
    assert np.abs(dec).max() <= 448
    assert np.all(np.abs(dec * s[:, None] - x) <= np.abs(x) * 2**-3 + s[:, None] * 2**-9)
    w, sw = oracle.fp8_quantize_rows((g.standard_normal((40, 9))).astype(np.float32).T.copy())
    wk = np.ascontiguousarray(w.T)
    out = oracle.fp8_gemm(q, s, wk, sw, 6, 40, 9)
    wdec = np.vectorize(oracle.e4m3_to_f32)(wk).astype(np.float64)
    want = (dec.astype(np.float64) @ wdec) * s[:, None] * sw[None, :]
    assert np.array_equal(out, _bf(want.astype(np.float32)))


def test_fused_moe_oracle_per_slot():
    g = np.random.default_rng(4)
    T, k, E, K, N, bs = 6, 2, 3, 16, 5, 4
    ids = g.integers(0, E, (T, k)).astype(np.int32)
    s, e, n = oracle.moe_align_block_size(ids, E, bs)
    A = _bf(g.standard_normal((T, K)))
    B = _bf(g.standard_normal((E, N, K)) * 0.1)
    bias = _bf(g.standard_normal((E, N)))
    C = oracle.fused_moe(A, B, None, None, bias, None, s, e, n, T, K, N, E, T * k, k, bs, 0)
    for slot in range(T * k):
        ex = ids.ravel()[slot]
        acc = synth.bf16_bits_to_f32(B[ex]).astype(np.float64) @ synth.bf16_bits_to_f32(A[slot // k]).astype(np.float64)
        want = _bf((acc.astype(np.float32) + synth.bf16_bits_to_f32(bias[ex])).astype(np.float32))
        assert np.array_equal(C[slot], want)
    # routed-weight variant on an already expanded A
    A2 = _bf(g.standard_normal((T * k, K)))
    tw = g.uniform(0, 1, T * k).astype(np.float32)
    Bq = g.integers(-127, 128, (E, N, K)).astype(np.int8)
    Bs = _bf(g.uniform(0.01, 0.02, (E, N)))
    C2 = oracle.fused_moe(A2, None, Bq, Bs, None, tw, s, e, n, T * k, K, N, E, T * k, k, bs, 1)
    for slot in range(T * k):
        ex = ids.ravel()[slot]
        acc = Bq[ex].astype(np.float64) @ synth.bf16_bits_to_f32(A2[slot]).astype(np.float64)
        acc = acc * synth.bf16_bits_to_f32(Bs[ex])
        want = _bf((acc.astype(np.float32) * tw[slot]).astype(np.float32))
        assert np.array_equal(C2[slot], want)


# ---------------------------------------------------------------- legacy MoE
def _bf(a):
    return oracle.f32_to_bf16(np.asarray(a, np.float32))


def test_oracle_moe_combine_closed_forms():
    # w = 1 with small integers: y + sum of the matching e rows, exactly;
    # slots with idx >= N or top >= topk change nothing
    N, M, topk = 4, 16, 2
    g = np.random.default_rng(1)
    y = g.integers(-8, 9, (N, M)).astype(np.float32)
    e = g.integers(-8, 9, (6, M)).astype(np.float32)
    idx = np.array([0, 2, 2, 7, 1, 3], np.uint32)
    top = np.array([0, 1, 0, 0, 5, 1], np.uint32)
    w = np.ones(N * topk, np.float32)
    got = oracle.bf16_to_f32(oracle.moe_combine(oracle.BF16, _bf(y), _bf(e), w, idx, top, N, 6, M, topk))
    want = y.copy()
    want[0] += e[0]
    want[2] += e[1] + e[2]
    want[3] += e[5]
    assert np.array_equal(got, want)
    # the routed weight scales its slot's row: w = 0.5 on an even row halves it
    w2 = np.full(N * topk, 0.5, np.float32)
    e2 = 2 * g.integers(-8, 9, (1, M)).astype(np.float32)
    got = oracle.bf16_to_f32(oracle.moe_combine(oracle.BF16, _bf(np.zeros((N, M))), _bf(e2), w2,
                                                np.array([1], np.uint32), np.array([1], np.uint32),
                                                N, 1, M, topk))
    assert np.array_equal(got[1], e2[0] / 2) and not got[[0, 2, 3]].any()


def test_oracle_moe_combine_rounds_per_slot():
    # two slots of 2^-8 into y = 1: each add rounds to bf16 on its own
    # (1 + 2^-8 is a tie that rounds to 1), so the result stays 1; summing
    # the slots first would give 1 + 2^-7
    N, M, topk = 1, 4, 2
    e = np.full((2, M), 2.0 ** -8, np.float32)
    got = oracle.moe_combine(oracle.BF16, _bf(np.ones((N, M))), _bf(e), np.ones(2, np.float32),
                             np.zeros(2, np.uint32), np.array([0, 1], np.uint32), N, 2, M, topk)
    assert np.array_equal(oracle.bf16_to_f32(got), np.ones((N, M), np.float32))
    # f16 (10-bit mantissa): 2^-8 is representable next to 1, so both land
    h = lambda a: np.asarray(a, np.float32).astype(np.float16).view(np.uint16)
    got16 = oracle.moe_combine(oracle.F16, h(np.ones((N, M))), h(e), np.ones(2, np.float32),
                               np.zeros(2, np.uint32), np.array([0, 1], np.uint32), N, 2, M, topk)
    assert np.array_equal(got16.view(np.float16).astype(np.float32),
                          np.full((N, M), 1 + 2.0 ** -7, np.float32))


@pytest.mark.parametrize("M", [1, 3])
def test_oracle_indexed_moe_integer_exact(M):
    # integer operands: out = W[e] . x exactly (numpy int64), with slot i
    # reading x[b, 0] when M == 1 and x[b, i] when M == topk; ids >= E keep
    # the marker already in out
    B, K, N, E, topk = 3, 64, 24, 4, 3
    g = np.random.default_rng(M)
    x = g.integers(-5, 6, (B, M, K))
    w = g.integers(-5, 6, (E, N, K))
    ii = np.array([[0, 3, 9], [2, 2, 1], [4, 1, 0]], np.uint32)
    out0 = np.full((B, topk, N), 3.0, np.float32)
    got = oracle.bf16_to_f32(oracle.indexed_moe(oracle.BF16, _bf(x), _bf(w), _bf(out0), ii, N, K, M,
                                                B, topk, E))
    for b in range(B):
        for i in range(topk):
            e = ii[b, i]
            want = out0[b, i] if e >= E else (w[e] @ x[b, 0 if M == 1 else i]).astype(np.float32)
            assert np.array_equal(got[b, i], oracle.bf16_to_f32(_bf(want))), (b, i)


def test_oracle_indexed_moe_f32_order():
    # random bf16 operands: the oracle equals a numpy f32 loop summing k in
    # order (the reference's moe_matmul, moe_host.cpp:325-355)
    B, K, N, E, topk, M = 2, 96, 8, 3, 2, 2
    g = np.random.default_rng(4)
    xb, wb = _bf(g.standard_normal((B, M, K))), _bf(g.standard_normal((E, N, K)))
    x, w = oracle.bf16_to_f32(xb), oracle.bf16_to_f32(wb)
    ii = np.array([[1, 2], [0, 1]], np.uint32)
    got = oracle.indexed_moe(oracle.BF16, xb, wb, np.zeros((B, topk, N), np.uint16), ii, N, K, M,
                             B, topk, E)
    for b in range(B):
        for i in range(topk):
            for n in range(N):
                a = np.float32(0)
                for k in range(K):
                    a = np.float32(a + np.float32(x[b, i, k] * w[ii[b, i], n, k]))
                assert got[b, i, n] == _bf(np.array([a]))[0]
