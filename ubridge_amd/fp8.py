"""fp8 (OCP e4m3fn) W8A8 GEMM: per-token activation scales x per-channel
weight scales, bf16 output.  The reference has no fp8 path; the operator
mirrors the quantized matmul calling convention (device buffers in, device
buffers out, stream last).  Weights are prepacked once from [K, N] to
[N, K] (K contiguous), the layout the MFMA B operand reads."""
import ctypes

import torch

from ._lib import check, lib, register
from .ops import _DT_CODE, _need_cuda, _ptr, stream_ptr

_vp, _i = ctypes.c_void_p, ctypes.c_int
register("ubridge_fp8_gemm", _i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp])
register("ubridge_fp8_transpose", _i, [_vp, _vp, _i, _i, _vp])
register("ubridge_fp8_quantize_rows", _i, [_vp, _i, _vp, _vp, _i, _i, _vp])


def quantize_rows(x, stream=None):
    """x [R, C] -> (e4m3 codes uint8 [R, C], f32 scales [R]), scale = amax/448."""
    _need_cuda(x)
    x = x.contiguous()
    R, C = x.shape
    q = torch.empty(R, C, dtype=torch.uint8, device=x.device)
    s = torch.empty(R, dtype=torch.float32, device=x.device)
    check(lib.ubridge_fp8_quantize_rows(_ptr(x), _DT_CODE[x.dtype], _ptr(q), _ptr(s), R, C,
                                        stream_ptr(stream)))
    return q, s


def prepack_weight(w_kn, stream=None):
    """e4m3 [K, N] -> [N, K] (one-time weight layout change)."""
    _need_cuda(w_kn)
    K, N = w_kn.shape
    out = torch.empty(N, K, dtype=torch.uint8, device=w_kn.device)
    check(lib.ubridge_fp8_transpose(_ptr(w_kn.contiguous()), _ptr(out), K, N, stream_ptr(stream)))
    return out


def gemm(a_q, a_scale, w_nk, w_scale, out=None, stream=None):
    """out[M, N] bf16 = (a_q[M,K] . w_nk[N,K]^T) * a_scale[M] * w_scale[N]."""
    _need_cuda(a_q, a_scale, w_nk, w_scale)
    M, K = a_q.shape
    N = w_nk.shape[0]
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=a_q.device)
    check(lib.ubridge_fp8_gemm(_ptr(a_q), _ptr(a_scale), _ptr(w_nk), _ptr(w_scale), _ptr(out), M, K,
                               N, stream_ptr(stream)))
    return out
