"""GPU parity of the MoE chain (routing, align, grouped expert GEMM, SiLU,
combine) against the CPU oracle, through the C ABI."""
import numpy as np
import pytest
import torch

import oracle
from conftest import rel_err
from ubridge_amd import moe, ops, synth

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,E,k,norm", [(256, 128, 8, True), (37, 64, 6, False), (5, 4096, 2, True),
                                        (3, 8, 8, True)])
def test_topk_softmax(dev, dtype, T, E, k, norm):
    logits = torch.randn(T, E, generator=torch.Generator().manual_seed(E + T)).to(dtype)
    w, ids = moe.topk_softmax(logits.to(dev), k, norm)
    dt = {torch.float32: oracle.F32, torch.bfloat16: oracle.BF16, torch.float16: oracle.F16}[dtype]
    arr = logits.numpy() if dtype == torch.float32 else logits.view(torch.int16).numpy().view(np.uint16)
    ow, oi = oracle.topk_softmax(arr, k, norm, dt)
    assert np.array_equal(ids.cpu().numpy(), oi)
    if dtype == torch.float32:
        assert np.abs(w.cpu().numpy() - ow).max() <= 2e-6 * max(1.0, np.abs(ow).max())
    else:
        # expf may differ from libm by an ulp; after rounding to 16 bits at most one ulp apart
        d = np.abs(_bits(w).astype(np.int32) - ow.astype(np.int32))
        assert d.max() <= 1


def test_topk_softmax_ties(dev):
    logits = torch.zeros(2, 16)
    logits[1, [3, 9, 12]] = 2.0
    w, ids = moe.topk_softmax(logits.to(dev), 4, False)
    assert ids[0].tolist() == [0, 1, 2, 3]
    assert ids[1].tolist()[:3] == [3, 9, 12]


@pytest.mark.parametrize("T,k,E,bs", [(256, 8, 128, 16), (256, 8, 128, 64), (7, 2, 5, 4),
                                      (1, 1, 3, 8), (600, 4, 256, 32), (64, 8, 1024, 16),
                                      (4096, 8, 128, 32), (3000, 6, 60, 16), (5000, 2, 1024, 8),
                                      (1000, 8, 7, 64), (700, 8, 128, 1)])
def test_moe_align_exact(dev, T, k, E, bs):
    ids = np.random.default_rng(T * E + bs).integers(0, E, (T, k)).astype(np.int32)
    s, e, n = moe.moe_align_block_size(torch.from_numpy(ids).to(dev), E, bs)
    os_, oe, on = oracle.moe_align_block_size(ids, E, bs)
    assert n.item() == on[0]
    assert np.array_equal(s.cpu().numpy(), os_)
    assert np.array_equal(e.cpu().numpy(), oe)


def test_moe_align_expert_map_real_tokens(dev):
    T, k, E, bs = 50, 4, 16, 8
    ids = np.random.default_rng(3).integers(0, E, (T, k)).astype(np.int32)
    emap = np.where(np.arange(E) % 3 == 0, -1, np.arange(E) // 2).astype(np.int32)
    s, e, n = moe.moe_align_block_size(torch.from_numpy(ids).to(dev), E, bs, real_token_num=31,
                                       expert_map=torch.from_numpy(emap).to(dev))
    os_, oe, on = oracle.moe_align_block_size(ids, E, bs, real_token_num=31, expert_map=emap)
    assert n.item() == on[0]
    assert np.array_equal(s.cpu().numpy(), os_) and np.array_equal(e.cpu().numpy(), oe)
    s0, e0, n0 = moe.moe_align_block_size(torch.from_numpy(ids).to(dev), E, bs, real_token_num=0)
    assert n0.item() == 0 and (s0.cpu().numpy() == T * k).all()


def test_moe_align_expert_map_real_tokens_large(dev):
    # the general kernel well past one chunk per wavefront: 8000 slots
    T, k, E, bs = 2000, 4, 64, 16
    ids = np.random.default_rng(4).integers(0, E, (T, k)).astype(np.int32)
    emap = np.where(np.arange(E) % 5 == 1, -1, (np.arange(E) * 7) % E).astype(np.int32)
    for rtn in (T, 1234):
        s, e, n = moe.moe_align_block_size(torch.from_numpy(ids).to(dev), E, bs,
                                           real_token_num=rtn,
                                           expert_map=torch.from_numpy(emap).to(dev))
        os_, oe, on = oracle.moe_align_block_size(ids, E, bs, real_token_num=rtn, expert_map=emap)
        assert n.item() == on[0]
        assert np.array_equal(s.cpu().numpy(), os_) and np.array_equal(e.cpu().numpy(), oe)


def test_moe_align_bad_ids_flagged(dev):
    ids = torch.tensor([[0, 1], [2, 9]], dtype=torch.int32, device=dev)
    s, e, n = moe.moe_align_block_size(ids, 4, 2)
    with pytest.raises(Exception):
        moe.device_error()
    assert n.item() == 0
    moe.device_error()  # cleared


def _align(ids, E, bs, dev):
    return moe.moe_align_block_size(torch.from_numpy(ids).to(dev), E, bs)


@pytest.mark.parametrize("mrw", [0, 1])
@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("bias", [False, True])
def test_fused_moe_vs_oracle(dev, mrw, q8, bias):
    T, k, E, K, N, bs = 40, 3, 8, 128, 96, 16
    g = np.random.default_rng(7 + mrw + 2 * q8)
    ids = g.integers(0, E, (T, k)).astype(np.int32)
    A = synth.bf16_activations(T * k if mrw else T, K, seed=1)
    if q8:
        Bq = g.integers(-127, 128, (E, N, K)).astype(np.int8)
        Bs = synth.f32_to_bf16_bits(g.uniform(0.002, 0.02, (E, N)).astype(np.float32))
        B = None
    else:
        B = synth.f32_to_bf16_bits((g.standard_normal((E, N, K)) * 0.05).astype(np.float32))
        Bq = Bs = None
    bv = synth.f32_to_bf16_bits(g.standard_normal((E, N)).astype(np.float32)) if bias else None
    tw = g.uniform(0, 1, T * k).astype(np.float32)
    s, e, n = _align(ids, E, bs, dev)
    bf = lambda x: torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(dev)
    C = torch.zeros(T * k, N, dtype=torch.bfloat16, device=dev)
    moe.invoke_fused_moe(bf(A), torch.from_numpy(Bq).to(dev) if q8 else bf(B), C,
                         torch.from_numpy(tw).to(dev) if mrw else None, s, e, n, k, bs, mrw,
                         B_scale=bf(Bs) if q8 else None, bias=bf(bv) if bias else None)
    want = oracle.fused_moe(A, B, Bq, Bs, bv, tw if mrw else None, s.cpu().numpy(), e.cpu().numpy(),
                            n.cpu().numpy(), A.shape[0], K, N, E, T * k, k, bs, mrw)
    got = oracle.bf16_to_f32(_bits(C))
    assert rel_err(got, oracle.bf16_to_f32(want)) < 1e-2


@pytest.mark.parametrize("K,N,bs,q8,mrw,dtype", [(384, 200, 16, True, 1, torch.bfloat16),
                                                  (640, 136, 64, False, 0, torch.bfloat16),
                                                  (416, 264, 32, True, 0, torch.float16),
                                                  (1024, 128, 4, False, 1, torch.float16)])
def test_fused_moe_multi_step(dev, K, N, bs, q8, mrw, dtype):
    # K > 256 (several K-steps through the load ring); several blocks per
    # expert, partial column tiles, a partial last K-step, experts mapped to
    # -1 (zero rows)
    T, k, E = 150, 4, 12
    g = np.random.default_rng(K + N + bs)
    ids = g.integers(0, E, (T, k)).astype(np.int32)
    emap = np.arange(E, dtype=np.int32)
    emap[[2, 7]] = -1
    s, e, n = moe.moe_align_block_size(torch.from_numpy(ids).to(dev), E, bs,
                                       expert_map=torch.from_numpy(emap).to(dev))
    A = torch.randn(T * k if mrw else T, K, device=dev).to(dtype)
    if q8:
        B = torch.randint(-127, 128, (E, N, K), device=dev, dtype=torch.int8)
        Bs = (torch.rand(E, N, device=dev) * 0.02 + 0.002).to(dtype)
        Bf = B.float() * Bs.float().unsqueeze(-1)
    else:
        B = (torch.randn(E, N, K, device=dev) * 0.05).to(dtype)
        Bs = None
        Bf = B.float()
    tw = torch.rand(T * k, device=dev)
    C = torch.full((T * k, N), 3.0, dtype=dtype, device=dev)
    moe.invoke_fused_moe(A, B, C, tw if mrw else None, s, e, n, k, bs, mrw, B_scale=Bs)
    ids_f = torch.from_numpy(ids.ravel()).long()
    em = torch.from_numpy(emap).long()[ids_f]
    arow = torch.arange(T * k) if mrw else torch.arange(T * k) // k
    want = torch.zeros(T * k, N, dtype=torch.float64)
    for slot in range(T * k):
        ex = int(em[slot])
        if ex < 0:
            continue
        v = A[arow[slot]].double() @ Bf[ex].double().T
        want[slot] = v * (float(tw[slot]) if mrw else 1.0)
    got = C.double().cpu()
    assert (got[em < 0] == 0).all()
    assert rel_err(got.numpy(), want.numpy()) < 1e-2


def test_fused_moe_expert_minus_one_zeroes(dev):
    T, k, E, K, N, bs = 10, 2, 4, 64, 32, 4
    ids = np.random.default_rng(5).integers(0, E, (T, k)).astype(np.int32)
    emap = np.array([0, -1, 2, -1], np.int32)
    s, e, n = moe.moe_align_block_size(torch.from_numpy(ids).to(dev), E, bs,
                                       expert_map=torch.from_numpy(emap).to(dev))
    A = torch.randn(T, K, device=dev).bfloat16()
    B = torch.randn(E, N, K, device=dev).bfloat16()
    C = torch.full((T * k, N), 7.0, dtype=torch.bfloat16, device=dev)
    moe.invoke_fused_moe(A, B, C, None, s, e, n, k, bs, False)
    ids_f = ids.ravel()
    for slot in range(T * k):
        row = C[slot].float()
        if emap[ids_f[slot]] == -1:
            assert (row == 0).all()
        else:
            want = A[slot // k].double() @ B[emap[ids_f[slot]]].double().T
            assert torch.allclose(row.double(), want, rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,E,k,bs,norm", [(256, 128, 8, 32, 1), (37, 60, 3, 16, 0), (5, 200, 6, 4, 1),
                                           (600, 64, 8, 64, 1), (1, 8, 2, 32, 0)])
def test_moe_route_matches_separate_ops(dev, dtype, T, E, k, bs, norm):
    # the routing call (small-slot align for T*k <= 4096, the general align
    # above) against topk_softmax_* + moe_align_block_size, bit for bit
    g = torch.Generator(device=dev).manual_seed(T * E + k)
    logits = torch.randn(T, E, device=dev, generator=g).to(dtype)
    w, wf, ids, s, e, n = moe.moe_route(logits, k, E, bs, bool(norm))
    w0, ids0 = moe.topk_softmax(logits, k, bool(norm))
    s0, e0, n0 = moe.moe_align_block_size(ids0, E, bs)
    assert torch.equal(ids, ids0)
    assert torch.equal(w.view(torch.int16 if dtype != torch.float32 else torch.int32),
                       w0.view(torch.int16 if dtype != torch.float32 else torch.int32))
    assert torch.equal(wf, w0.float())
    assert int(n) == int(n0)
    assert torch.equal(s, s0) and torch.equal(e, e0)
    dt = {torch.float32: oracle.F32, torch.bfloat16: oracle.BF16, torch.float16: oracle.F16}[dtype]
    lc = logits.cpu()
    arr = lc.numpy() if dtype == torch.float32 else lc.view(torch.int16).numpy().view(np.uint16)
    _, oi = oracle.topk_softmax(arr, k, norm, dt)
    assert np.array_equal(ids.cpu().numpy(), oi)
    os_, oe, on = oracle.moe_align_block_size(oi, E, bs)
    assert int(n) == int(on[0]) and np.array_equal(s.cpu().numpy(), os_)


def test_silu_and_mul_and_sum(dev):
    x = torch.randn(33, 2 * 48, device=dev).bfloat16()
    out = moe.silu_and_mul(x)
    xf = x.float()
    want = (torch.nn.functional.silu(xf[:, :48]) * xf[:, 48:]).bfloat16()
    assert (out.float() - want.float()).abs().max().item() <= 1e-2 * want.float().abs().max().item()
    y = torch.randn(12 * 4, 40, device=dev).bfloat16()
    s = moe.moe_sum(y, 12, 4)
    assert torch.allclose(s.float(), y.float().view(12, 4, 40).sum(1), rtol=1e-2, atol=1e-2)


def test_full_chain_cfg4(dev):
    # 256 tokens, hidden 2048, 128 experts, top-8, gate/up 2048->1536, down 768->2048
    T, H, E, k, I = 256, 2048, 128, 8, 768
    g = torch.Generator(device=dev).manual_seed(4)
    x = torch.randn(T, H, device=dev, generator=g).bfloat16()
    logits = torch.randn(T, E, device=dev, generator=g).bfloat16()
    w13 = torch.randint(-127, 128, (E, 2 * I, H), device=dev, dtype=torch.int8, generator=g)
    s13 = (torch.rand(E, 2 * I, device=dev, generator=g) * 0.002 + 0.0002).bfloat16()
    w2 = torch.randint(-127, 128, (E, H, I), device=dev, dtype=torch.int8, generator=g)
    s2 = (torch.rand(E, H, device=dev, generator=g) * 0.002 + 0.0002).bfloat16()
    layer = moe.FusedMoE(w13, w2, s13, s2, topk=k, renormalize=True, block_size=32)
    out = layer(x, logits)
    moe.device_error()
    # reference: same routing (checked above against the oracle), f32 math per token
    w, ids = moe.topk_softmax(logits, k, True)
    ref = torch.zeros(T, H, dtype=torch.float64, device=dev)
    xf = x.double()
    for e in range(E):
        tok, slot = (ids == e).nonzero(as_tuple=True)
        if tok.numel() == 0:
            continue
        h = xf[tok] @ (w13[e].double() * s13[e].double()[:, None]).T
        h = h.bfloat16().double()
        act = (torch.nn.functional.silu(h[:, :I]) * h[:, I:]).bfloat16().double()
        o = act @ (w2[e].double() * s2[e].double()[:, None]).T
        ref.index_add_(0, tok, o * w[tok, slot].double()[:, None])
    err = (torch.linalg.norm(out.double() - ref) / torch.linalg.norm(ref)).item()
    assert err < 2e-2, err


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_legacy_moe_combine_vs_oracle(dev, dtype):
    # moe_{bf16,f16}: rows hit by several slots (accumulated in slot order),
    # out-of-range row ids and top slots (skipped); bit-exact with the oracle
    N, M, topk, K = 6, 300, 2, 12
    g = torch.Generator().manual_seed(3)
    y = torch.randn(N, M, generator=g).to(dtype)
    e_out = torch.randn(K, M, generator=g).to(dtype)
    w = torch.rand(N * topk, generator=g)
    idx = torch.tensor([0, 1, 1, 5, 9, 2, 0, 3, 4, 1, 1, 6], dtype=torch.int32)
    top = torch.tensor([0, 1, 0, 1, 0, 2, 1, 0, 1, 1, 0, 0], dtype=torch.int32)
    dt = oracle.BF16 if dtype == torch.bfloat16 else oracle.F16
    want = oracle.moe_combine(dt, y.view(torch.int16).numpy().view(np.uint16).copy(),
                              e_out.view(torch.int16).numpy().view(np.uint16), w.numpy(),
                              idx.numpy().view(np.uint32), top.numpy().view(np.uint32), N, K, M,
                              topk)
    got = moe.moe_combine(y.to(dev), e_out.to(dev), w.to(dev), idx.to(dev), top.to(dev), topk)
    assert np.array_equal(got.cpu().view(torch.int16).numpy().view(np.uint16), want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M", [1, 3])
def test_legacy_indexed_moe_vs_oracle(dev, dtype, M):
    # indexed_moe_{bf16,f16}: M == 1 (every slot reads x[b, 0]) and M == topk
    # (slot i reads x[b, i]); expert ids >= E leave their output rows as they
    # were (pre-filled with a marker)
    B, K, N, E, topk = 4, 256, 80, 5, 3
    g = torch.Generator().manual_seed(M)
    x = torch.randn(B, M, K, generator=g).to(dtype)
    we = torch.randn(E, N, K, generator=g).to(dtype)
    ii = torch.tensor([[0, 4, 7], [2, 2, 1], [1, 3, 5], [4, 0, 2]], dtype=torch.int32)
    out0 = torch.full((B, topk, N), 3.0, dtype=dtype)
    dt = oracle.BF16 if dtype == torch.bfloat16 else oracle.F16
    u16 = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
    want = oracle.indexed_moe(dt, u16(x), u16(we), u16(out0), ii.numpy().view(np.uint32), N, K, M,
                              B, topk, E)
    got = moe.indexed_moe(x.to(dev), we.to(dev), ii.to(dev), out=out0.to(dev))
    got = u16(got.cpu())
    # same f32 sum order and roundings as the oracle: bit-exact
    assert np.array_equal(got, want)
    gf = torch.from_numpy(got.view(np.int16)).view(dtype).float()
    assert torch.equal(gf[0, 2], torch.full((N,), 3.0)) and torch.equal(gf[2, 2], gf[0, 2])


def test_legacy_indexed_moe_exact(dev):
    # integer-valued operands: f32 sums are exact, so the GPU equals the
    # oracle bit for bit (M = topk, so each slot reads its own input row)
    B, K, N, E, topk = 2, 128, 64, 3, 2
    g = torch.Generator().manual_seed(9)
    x = torch.randint(-4, 5, (B, topk, K), generator=g).bfloat16()
    we = torch.randint(-4, 5, (E, N, K), generator=g).bfloat16()
    ii = torch.tensor([[2, 0], [1, 1]], dtype=torch.int32)
    got = moe.indexed_moe(x.to(dev), we.to(dev), ii.to(dev)).cpu()
    u16 = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
    want = oracle.indexed_moe(oracle.BF16, u16(x), u16(we), np.zeros((B, topk, N), np.uint16),
                              ii.numpy().view(np.uint32), N, K, topk, B, topk, E)
    assert np.array_equal(u16(got), want)


@pytest.mark.parametrize("T,k,E,K,I,bs,dtype,emap", [
    (256, 8, 128, 2048, 768, 32, torch.bfloat16, False),   # configs[3] gate/up
    (37, 3, 8, 416, 72, 16, torch.bfloat16, True),          # partial column tile, -1 experts
    (64, 4, 16, 256, 200, 64, torch.float16, False),        # several 32-row sub-blocks
    (9, 2, 4, 96, 40, 4, torch.bfloat16, True),             # bs % 4 == 0, tiny
    (20, 2, 6, 128, 64, 6, torch.float16, False),           # bs % 4 != 0: plain row loads
])
def test_fused_gate_up_silu_matches_two_calls(dev, T, k, E, K, I, bs, dtype, emap):
    g = torch.Generator(device="cpu").manual_seed(T + K + I)
    ids = torch.randint(0, E, (T, k), generator=g, dtype=torch.int32)
    em = None
    if emap:
        m = torch.arange(E, dtype=torch.int32)
        m[1::3] = -1
        em = m.to(dev)
    s, e, n = moe.moe_align_block_size(ids.to(dev), E, bs, expert_map=em)
    x = torch.randn(T, K, generator=g).to(dtype).to(dev)
    w13 = torch.randint(-127, 128, (E, 2 * I, K), generator=g, dtype=torch.int8).to(dev)
    s13 = (torch.rand(E, 2 * I, generator=g) * 0.01 + 0.001).to(dtype).to(dev)
    h1 = torch.zeros(T * k, 2 * I, dtype=dtype, device=dev)
    moe.invoke_fused_moe(x, w13, h1, None, s, e, n, k, bs, False, B_scale=s13)
    want = moe.silu_and_mul(h1)
    got = torch.full((T * k, I), 7.0, dtype=dtype, device=dev)
    moe.fused_moe_gate_up_silu(x, w13, s13, s, e, n, k, bs, out=got)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("N,dtype", [(40, torch.bfloat16), (36, torch.bfloat16), (2048, torch.float16)])
def test_moe_sum_bits(dev, N, dtype):
    # f32 accumulation in slot order, one rounding: bit for bit (the 8-column
    # vector kernel for N % 8 == 0, the scalar one otherwise)
    T, k = 13, 8
    y = torch.randn(T * k, N, device=dev).to(dtype)
    got = moe.moe_sum(y, T, k)
    yf = y.float().cpu().view(T, k, N)
    acc = yf[:, 0].clone()
    for j in range(1, k):
        acc = acc + yf[:, j]
    assert torch.equal(got.cpu().view(torch.int16), acc.to(dtype).view(torch.int16))


@pytest.mark.parametrize("T,k,E,K,N,bs,dtype,emap,path", [
    (256, 8, 128, 768, 2048, 32, torch.bfloat16, False, 0),  # configs[3] down projection
    (37, 3, 8, 416, 72, 16, torch.bfloat16, True, 0),        # partial column tile, -1 experts
    (64, 4, 16, 256, 200, 64, torch.float16, False, 0),      # several 32-row sub-blocks
    (9, 2, 4, 96, 40, 4, torch.bfloat16, True, 6),           # 64-column tiles, tiny
    (20, 2, 6, 128, 64, 6, torch.float16, False, 2),         # bs % 4 != 0, 256-column tiles
    (50, 6, 12, 192, 320, 32, torch.bfloat16, False, 9),     # 64 columns, BK 128
])
def test_fused_down_combine_matches_two_calls(dev, T, k, E, K, N, bs, dtype, emap, path):
    # down GEMM + moe_sum in one call: C and the combined output bit for bit
    # against the two operators, over the GEMM's tile variants
    g = torch.Generator(device="cpu").manual_seed(T + K + N)
    ids = torch.randint(0, E, (T, k), generator=g, dtype=torch.int32)
    em = None
    if emap:
        m = torch.arange(E, dtype=torch.int32)
        m[1::3] = -1
        em = m.to(dev)
    s, e, n = moe.moe_align_block_size(ids.to(dev), E, bs, expert_map=em)
    w = torch.rand(T, k, generator=g).to(dev)
    w2 = torch.randint(-127, 128, (E, N, K), generator=g, dtype=torch.int8).to(dev)
    s2 = (torch.rand(E, N, generator=g) * 0.01 + 0.001).to(dtype).to(dev)
    ops.tune_set("moe_gemm_path", path)
    try:
        for it in range(2):
            x = torch.randn(T * k, K, generator=g).to(dtype).to(dev)
            h = torch.zeros(T * k, N, dtype=dtype, device=dev)
            moe.invoke_fused_moe(x, w2, h, w.reshape(-1), s, e, n, k, bs, True, B_scale=s2)
            want = moe.moe_sum(h, T, k)
            hc = torch.full((T * k, N), 7.0, dtype=dtype, device=dev)
            got = moe.fused_moe_down_combine(x, w2, s2, w.reshape(-1), s, e, n, k, bs, C=hc)
            torch.cuda.synchronize()
            assert torch.equal(hc.view(torch.int16), h.view(torch.int16)), it
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), it
    finally:
        ops.tune_set("moe_gemm_path", 0)
    moe.device_error()


# ---- status-returning trio (kernels/topsaten_moe_wrapper.cpp:80-216)

@pytest.mark.parametrize("T,E,k,norm", [(256, 128, 8, 1), (37, 60, 3, 0), (5, 1024, 6, 1)])
def test_topsaten_topk_softmax(dev, T, E, k, norm):
    logits = torch.randn(T, E, generator=torch.Generator().manual_seed(T + 3 * E))
    w, ids, tei = moe.topsaten_topk_softmax(logits.to(dev), k, norm)
    w0, ids0 = moe.topk_softmax(logits.to(dev), k, bool(norm))
    assert torch.equal(ids, ids0) and torch.equal(w.view(torch.int32), w0.view(torch.int32))
    ow, oi = oracle.topk_softmax(logits.numpy(), k, norm, oracle.F32)
    assert np.array_equal(ids.cpu().numpy(), oi)
    want = np.arange(k)[None, :] * T + np.arange(T)[:, None]
    assert np.array_equal(tei.cpu().numpy(), want)


@pytest.mark.parametrize("T,k,E,bs", [(256, 8, 128, 16), (7, 2, 5, 4), (3000, 6, 60, 16)])
def test_topsaten_moe_align(dev, T, k, E, bs):
    ids = np.random.default_rng(T + E).integers(0, E, (T, k)).astype(np.int32)
    s, e, n = moe.topsaten_moe_align_block_size(torch.from_numpy(ids).to(dev), E, bs)
    os_, oe, on = oracle.moe_align_block_size(ids, E, bs)
    assert n.item() == on[0]
    assert np.array_equal(s.cpu().numpy(), os_) and np.array_equal(e.cpu().numpy(), oe)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mrw", [0, 1])
def test_topsaten_fused_moe_gemm(dev, dtype, mrw):
    # C [T, k, inter] with A [T, hidden] read at row t for every slot of token
    # t; the same bits as invoke_fused_moe on A (mrw 0) or on A repeated per
    # slot (mrw 1, whose reference form reads one A row per slot)
    T, k, E, K, N, bs = 45, 4, 8, 256, 160, 16
    g = torch.Generator().manual_seed(11 + mrw)
    A = (torch.randn(T, K, generator=g) * 0.5).to(dtype).to(dev)
    B = (torch.randn(E, N, K, generator=g) * 0.05).to(dtype).to(dev)
    logits = torch.randn(T, E, generator=g).to(dev)
    tw, ids, _ = moe.topsaten_topk_softmax(logits, k, 1)
    s, e, n = moe.topsaten_moe_align_block_size(ids, E, bs)
    C = moe.topsaten_fused_moe_gemm(A, B, tw, ids, s, e, n, mrw, bs)
    assert C.shape == (T, k, N)
    A0 = A.repeat_interleave(k, dim=0) if mrw else A
    C0 = torch.zeros(T * k, N, dtype=dtype, device=dev)
    moe.invoke_fused_moe(A0, B, C0, tw if mrw else None, s, e, n, k, bs, mrw)
    assert torch.equal(C.reshape(T * k, N).view(torch.int16), C0.view(torch.int16))
    # and against the CPU oracle of the grouped GEMM
    if dtype == torch.bfloat16:
        bits = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16)
        want = oracle.fused_moe(bits(A0), bits(B), None, None, None,
                                tw.cpu().numpy().reshape(-1) if mrw else None, s.cpu().numpy(),
                                e.cpu().numpy(), n.cpu().numpy(), A0.shape[0], K, N, E, T * k, k,
                                bs, mrw)
        got = oracle.bf16_to_f32(bits(C.reshape(T * k, N)))
        assert rel_err(got, oracle.bf16_to_f32(want)) < 1e-2
