"""GPU test of ubridge_qmatmul_noalloc (the allocation-free QMatMul): two
calls in a row through the C ABI, the second with a smaller input, each
compared with ubridge_qmatmul on a caller workspace.  Both run the same
kernels, so the outputs must be bit-identical."""
import ctypes

import numpy as np
import pytest
import torch

from ubridge_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu

_vp, _i, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
noalloc = _lib.register("ubridge_qmatmul_noalloc", _i, [_i, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp])
max_ws = _lib.register("ubridge_qmatmul_noalloc_max_workspace", _sz, [])


def _both(dev, qt, M, N, K, seed):
    w = torch.from_numpy(synth.make_weight_soa(qt, N, K, seed=seed)).to(dev)
    x = torch.from_numpy(synth.make_activations(M, K, seed=seed)).to(dev)
    y_ref = torch.empty(M, N, dtype=torch.float32, device=dev)
    y_na = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    wsb = _lib.lib.ubridge_qmatmul_workspace_size(qt, M, K)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    _lib.check(_lib.lib.ubridge_qmatmul(qt, w.data_ptr(), x.data_ptr(), 0, y_ref.data_ptr(), 0,
                                        M, N, K, ws.data_ptr(), wsb, s))
    print(f"noalloc qt={qt} M={M} N={N} K={K}", flush=True)
    _lib.check(noalloc(qt, w.data_ptr(), x.data_ptr(), 0, y_na.data_ptr(), 0, M, N, K, s))
    torch.cuda.synchronize()
    return y_ref.cpu().numpy(), y_na.cpu().numpy()


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0, ops.Q4_K])
def test_noalloc_matches_workspace_entry(dev, qt):
    # first call: 16 tokens (two-launch path through the scratch array);
    # second, smaller: 3 tokens, then 1 token (one-launch path)
    for M, N, K in ((16, 768, 4096), (3, 512, 2048), (1, 256, 1024)):
        a, b = _both(dev, qt, M, N, K, seed=M * 7 + qt)
        assert np.array_equal(a, b), f"qt={qt} M={M}: noalloc differs from ubridge_qmatmul"


def test_noalloc_rejects_oversize(dev):
    K = 14336
    M = int(max_ws() // K) + 1  # workspace > 1 byte per element: too big
    y = torch.empty(M, 16, device=dev)
    rc = noalloc(ops.Q8_0, 0, 0, 0, y.data_ptr(), 0, M, 16, K, None)
    assert rc == 1 and _lib.lib.ubridge_last_error() == 1


@pytest.mark.parametrize("qt", [ops.Q4_0, ops.Q8_0, ops.Q4_K])
def test_noalloc_prefill_allocates_nothing(dev, qt):
    # prefill sizes without a library workspace or hipBLASLt plan: the
    # pipelined GEMM dequantizing the GGUF blocks in registers, which
    # ubridge_qmatmul also takes below 768 tokens (bit-equal there when it
    # does not split K over workgroups into its stream workspace; at 128
    # tokens it does: GEMM tolerance).  Under knob w4a16_path = 1 both run the GEMM dequantizing
    # into LDS (bit-equal).
    K, N = 1024, 256
    for M in (512, 64):  # 64: the 64-row tiles
        ops.tune_set("w4a16_path", 7)  # ubridge_qmatmul without the K split it could add
        try:
            ref, na = _both(dev, qt, M, N, K, seed=11)
        finally:
            ops.tune_set("w4a16_path", 0)
        assert np.array_equal(ref, na)
    ref, na = _both(dev, qt, 512, N, K, seed=11)  # with it: f32 sums in another order
    assert np.linalg.norm(ref - na) / np.linalg.norm(ref) < 1e-5
    ref, na = _both(dev, qt, 128, N, K, seed=12)
    assert np.linalg.norm(ref - na) / np.linalg.norm(ref) < 4e-3
    ops.tune_set("w4a16_path", 1)
    try:
        ref1, na1 = _both(dev, qt, 128, N, K, seed=13)
    finally:
        ops.tune_set("w4a16_path", 0)
    assert np.array_equal(ref1, na1)
