"""GPU parity of the GGUF dequant / quantize kernels against the CPU oracle:
bit-exact on every output dtype, through the C ABI (ubridge_amd.ops wraps
the extern "C" entry points; the registry path goes through
ubridge_get_function / ubridge_launch)."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from ubridge_amd import ops, registry, synth

pytestmark = pytest.mark.gpu

DT = {torch.float32: oracle.F32, torch.float16: oracle.F16, torch.bfloat16: oracle.BF16}


def _bits(t):
    t = t.cpu()
    return t.view(torch.int32).numpy() if t.dtype == torch.float32 else t.view(torch.int16).numpy()


def _want_bits(a):
    return a.view(np.int32) if a.dtype == np.float32 else a.view(np.int16)


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0, ops.Q4_K])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N,K", [(64, 512), (3, 256), (1, 4096)])
def test_dequant_bit_exact(dev, qt, dtype, N, K):
    w = synth.make_weight_soa(qt, N, K, seed=N * 7 + K)
    got = ops.dequantize_block(qt, torch.from_numpy(w).to(dev), N * K, dtype)
    want = oracle.dequant(qt, w, N * K, DT[dtype])
    assert np.array_equal(_bits(got), _want_bits(want))


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0])
def test_dequant_odd_block_count_fallback(dev, qt):
    # 3 blocks: the payload starts at byte 6, not 16-aligned
    w = synth.make_weight_soa(qt, 1, 96, seed=5)
    for dtype in (torch.float32, torch.bfloat16):
        got = ops.dequantize_block(qt, torch.from_numpy(w).to(dev), 96, dtype)
        assert np.array_equal(_bits(got), _want_bits(oracle.dequant(qt, w, 96, DT[dtype])))


def test_dequant_golden(dev, golden):
    for name, qt in (("q8_0", ops.Q8_0), ("q4_0", ops.Q4_0), ("q4_k", ops.Q4_K)):
        soa = torch.from_numpy(golden[f"{name}_soa"]).to(dev)
        for dtype, suf in ((torch.float32, "f32"), (torch.float16, "f16"), (torch.bfloat16, "bf16")):
            want = golden[f"{name}_{suf}"]
            got = ops.dequantize_block(qt, soa, want.size, dtype)
            assert np.array_equal(_bits(got), _want_bits(want)), (name, suf)


def test_dequant_full_size_checksum(dev):
    # Llama-3-8B fused gate/up, Q4_K: bit-exact on the whole 117M-element tensor
    N, K = 28672, 4096
    w = synth.make_weight_soa(ops.Q4_K, N, K, seed=99)
    got = ops.dequantize_block(ops.Q4_K, torch.from_numpy(w).to(dev), N * K, torch.float32)
    want = oracle.dequant(oracle.Q4_K, w, N * K, oracle.F32)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_dequant_empty(dev):
    w = torch.zeros(16, dtype=torch.uint8, device=dev)
    out = ops.dequantize_block(ops.Q8_0, w, 0, torch.float32)
    assert out.numel() == 0


def test_registry_launch(dev):
    N, K = 16, 256
    w = synth.make_weight_soa(ops.Q8_0, N, K, seed=1)
    wt = torch.from_numpy(w).to(dev)
    out = torch.empty(N * K, dtype=torch.bfloat16, device=dev)
    f = registry.get_function("dequantize_block_q8_0_bf16", "quant")
    f.launch((ctypes.c_void_p(wt.data_ptr()), ctypes.c_void_p(out.data_ptr()),
              ctypes.c_size_t(N * K)))
    assert np.array_equal(_bits(out), _want_bits(oracle.dequant(ops.Q8_0, w, N * K, oracle.BF16)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape,shift", [((3, 1024), 0), ((1, 96), 0), ((3, 1024), 1),
                                         ((64, 4096), 0)])
def test_quantize_block_q8_0(dev, dtype, shape, shift):
    # eight lanes per block (aligned input, even block count) or one lane per
    # block (3 blocks: the codes start 2-byte aligned; input one element off)
    x = synth.make_activations(*shape, seed=4)
    x[0, :32] = 0.0
    xt = torch.from_numpy(x).to(dtype)
    buf = torch.zeros(xt.numel() + 8, dtype=dtype, device=dev)
    xd = buf[shift:shift + xt.numel()]
    xd.copy_(xt.reshape(-1).to(dev))
    got = ops.quantize_block_q8_0(xd).cpu().numpy()
    want = oracle.quantize_q8_0(xt.float().numpy())
    assert np.array_equal(got, want)


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0, ops.Q4_K])
@pytest.mark.parametrize("N,K", [(32, 1024), (4096, 4096)])
def test_gguf_soa_roundtrip(dev, qt, N, K):
    w = synth.make_weight_soa(qt, N, K, seed=8)
    nb = N * K // ops.BLOCK[qt]
    aos = oracle.soa_to_aos(qt, w, nb)
    got = ops.gguf_to_soa(qt, torch.from_numpy(aos).to(dev))
    assert np.array_equal(got.cpu().numpy(), w)
    back = ops.soa_to_gguf(qt, got)
    assert np.array_equal(back.cpu().numpy(), aos)
