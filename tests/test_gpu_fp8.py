"""GPU parity of the fp8 W8A8 path (row quantization, weight prepack, MFMA
GEMM) against the CPU oracle; tolerance rel-err <= 2e-2 as the north star
states for fp8 (the oracle accumulates the decoded products in f64)."""
import numpy as np
import pytest
import torch

import oracle
from conftest import rel_err
from ubridge_amd import fp8, ops

pytestmark = pytest.mark.gpu


def test_quantize_rows_bit_exact(dev):
    x = torch.randn(37, 1000, generator=torch.Generator().manual_seed(1))
    x[3] = 0.0
    x[5, 7] = 1e-9
    q, s = fp8.quantize_rows(x.to(dev))
    oq, os_ = oracle.fp8_quantize_rows(x.numpy())
    assert np.array_equal(s.cpu().numpy(), os_)
    assert np.array_equal(q.cpu().numpy(), oq)
    # bf16 input
    xb = x.bfloat16()
    q2, s2 = fp8.quantize_rows(xb.to(dev))
    oq2, os2 = oracle.fp8_quantize_rows(xb.float().numpy())
    assert np.array_equal(q2.cpu().numpy(), oq2) and np.array_equal(s2.cpu().numpy(), os2)


def test_prepack_transpose(dev):
    w = torch.randint(0, 256, (200, 72), dtype=torch.uint8, device=dev)
    assert torch.equal(fp8.prepack_weight(w), w.T.contiguous())


@pytest.fixture(params=[0, 3, 2, 4], ids=["default", "own_bk128", "4_waves", "8_waves_bk64"])
def fp8_variant(request):
    # gemm_tile knob: 0 the default (hipBLASLt's fp8 GEMM with row / column
    # scale vectors where it serves the shape, else the kernel of 3), 3 the
    # library's own kernel (128-byte K-steps when K % 128 == 0, else 64-byte
    # ones), 2 its 4-wavefront kernel, 4 the 8-wavefront 64-byte one
    ops.tune_set("gemm_tile", request.param)
    yield request.param
    ops.tune_set("gemm_tile", 0)


@pytest.mark.parametrize("M,K,N", [(64, 256, 128), (130, 512, 200), (1, 128, 40), (257, 384, 384),
                                   (300, 64, 520), (40, 1216, 264)])
def test_fp8_gemm_vs_oracle(dev, fp8_variant, M, K, N):
    g = torch.Generator().manual_seed(M + K + N)
    a = torch.randn(M, K, generator=g)
    w = torch.randn(K, N, generator=g)
    aq, sa = oracle.fp8_quantize_rows(a.numpy())
    wq_t, sw = oracle.fp8_quantize_rows(w.numpy().T.copy())  # per output channel n
    wq = np.ascontiguousarray(wq_t.T)  # [K, N] as the config stores it
    w_nk = fp8.prepack_weight(torch.from_numpy(wq).to(dev))
    out = fp8.gemm(torch.from_numpy(aq).to(dev), torch.from_numpy(sa).to(dev), w_nk,
                   torch.from_numpy(sw).to(dev))
    want = oracle.fp8_gemm(aq, sa, wq, sw, M, K, N, nthreads=8)
    got = out.float().cpu().numpy()
    assert rel_err(got, oracle.bf16_to_f32(want)) < 2e-2
    # and against the unquantized product: fp8 quantization error is bounded
    assert rel_err(got, a.double().numpy() @ w.double().numpy()) < 8e-2


@pytest.mark.parametrize("M", [256, 4096])
def test_fp8_cfg5(dev, fp8_variant, M):
    # configs[4] shapes K=8192, N=28672; M = 4096 is the full config (16 row
    # tiles, so the XCD-grouped tile order is exercised), checked against the
    # f64 product of the decoded operands, globally and per 256-row band
    K, N = 8192, 28672
    gen = torch.Generator(device=dev).manual_seed(5)
    a = torch.randn(M, K, device=dev, generator=gen)
    w = torch.randn(K, N, device=dev, generator=gen)
    aq, sa = fp8.quantize_rows(a)
    wq_nk, sw = fp8.quantize_rows(w.T.contiguous())
    out = fp8.gemm(aq, sa, wq_nk, sw)
    dec = lambda q: q.view(torch.float8_e4m3fn).double()
    want = (dec(aq) * sa.double()[:, None]) @ (dec(wq_nk) * sw.double()[:, None]).T
    err = (torch.linalg.norm(out.double() - want) / torch.linalg.norm(want)).item()
    assert err < 2e-2, err
    band = [(torch.linalg.norm(out[i:i + 256].double() - want[i:i + 256]) /
             torch.linalg.norm(want[i:i + 256])).item() for i in range(0, M, 256)]
    assert max(band) < 2e-2, band
