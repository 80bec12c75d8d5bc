"""Host-side mirror of Ubridge's quantized-matmul operator interface.

Every function here is a thin torch-facing wrapper over one C-ABI entry point
of libubridge_hip.so (include/ubridge_hip.h).  torch only supplies device
memory and the current HIP stream; all arithmetic runs in the HIP kernels.
Names and argument meanings follow the reference's operators:
  dequantize_block_{q8_0,q4_k}_{f16,bf16,f32}  kernels/quant.cpp:257-268,477-488
  quantize_block_q8_0_{bf16,f16,f32}           kernels/quant.cpp:331-353
  QMatMul (Candle's quantized matmul), served on the reference by dequant +
  matmul_bf16 (kernels/matmul.cpp:1143-1184), here by the fused GEMV.
"""
import ctypes

import torch

from . import _lib
from ._lib import check, lib

Q4_0, Q8_0, Q4_K = 2, 8, 12
F32, F16, BF16 = 0, 1, 2
BLOCK = {Q4_0: 32, Q8_0: 32, Q4_K: 256}
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34, Q4_K: 144}
_DT_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}
_DT_NAME = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}
_Q_NAME = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k"}


def stream_ptr(stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _need_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("ubridge_amd ops take device tensors")


def quant_bytes(qtype, numel):
    """Bytes of a SoA-packed tensor with numel elements."""
    return numel // BLOCK[qtype] * BLOCK_BYTES[qtype]


# ----------------------------------------------------------------- dequant
def dequantize_block(qtype, w, numel, dtype=torch.bfloat16, out=None, stream=None):
    """Dequantize a SoA block tensor (uint8, reference layout) to dtype."""
    _need_cuda(w)
    if out is None:
        out = torch.empty(numel, dtype=dtype, device=w.device)
    fn = getattr(lib, f"dequantize_block_{_Q_NAME[qtype]}_{_DT_NAME[out.dtype]}")
    fn(_ptr(w), _ptr(out), numel, stream_ptr(stream))
    check()
    return out


def quantize_block_q8_0(x, out=None, stream=None):
    """Quantize x (f32/f16/bf16) to SoA Q8_0 bytes (quantize_block_q8_0_*)."""
    _need_cuda(x)
    x = x.contiguous()
    n = x.numel()
    if out is None:
        out = torch.empty(n // 32 * 34, dtype=torch.uint8, device=x.device)
    fn = getattr(lib, f"quantize_block_q8_0_{_DT_NAME[x.dtype]}")
    fn(_ptr(x), _ptr(out), n * x.element_size(), out.numel(), stream_ptr(stream))
    check()
    return out


def gguf_to_soa(qtype, aos, stream=None):
    _need_cuda(aos)
    out = torch.empty_like(aos)
    nb = aos.numel() // BLOCK_BYTES[qtype]
    check(lib.ubridge_gguf_to_soa(qtype, _ptr(aos), _ptr(out), nb, stream_ptr(stream)))
    return out


def soa_to_gguf(qtype, soa, stream=None):
    _need_cuda(soa)
    out = torch.empty_like(soa)
    nb = soa.numel() // BLOCK_BYTES[qtype]
    check(lib.ubridge_soa_to_gguf(qtype, _ptr(soa), _ptr(out), nb, stream_ptr(stream)))
    return out


# ----------------------------------------------------------------- QMatMul
class QMatMul:
    """Candle-style quantized matmul: y = x @ W^T with W [N, K] GGUF-quantized.

    w is the SoA uint8 device tensor (reference layout).  x is f32 or bf16
    [..., K]; the result is f32 (Candle's CPU QMatMul output) unless
    out_dtype=torch.bfloat16.
    """

    def __init__(self, qtype, w, N, K):
        _need_cuda(w)
        if w.numel() != quant_bytes(qtype, N * K):
            raise ValueError(f"weight holds {w.numel()} bytes, expected {quant_bytes(qtype, N * K)}")
        self.qtype, self.w, self.N, self.K = qtype, w, N, K
        self._ws = None

    def workspace(self, M):
        need = lib.ubridge_qmatmul_workspace_size(self.qtype, M, self.K)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(max(need, 1), dtype=torch.uint8, device=self.w.device)
        return self._ws

    def quantize(self, x, stream=None):
        x2 = x.reshape(-1, self.K).contiguous()
        M = x2.shape[0]
        ws = self.workspace(M)
        check(lib.ubridge_quantize_activations(self.qtype, _ptr(x2), _DT_CODE[x2.dtype], M, self.K,
                                               _ptr(ws), ws.numel(), stream_ptr(stream)))
        return M

    def matmul_prequantized(self, M, out, stream=None):
        check(lib.ubridge_qmatmul_prequantized(self.qtype, _ptr(self.w), _ptr(out),
                                               _DT_CODE[out.dtype], M, self.N, self.K,
                                               _ptr(self._ws), stream_ptr(stream)))
        return out

    def forward(self, x, out_dtype=torch.float32, out=None, stream=None):
        _need_cuda(x)
        if x.dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("QMatMul takes f32 or bf16 activations")
        x2 = x.reshape(-1, self.K).contiguous()
        M = x2.shape[0]
        if out is None:
            out = torch.empty(M, self.N, dtype=out_dtype, device=x.device)
        ws = self.workspace(M)
        check(lib.ubridge_qmatmul(self.qtype, _ptr(self.w), _ptr(x2), _DT_CODE[x2.dtype],
                                  _ptr(out), _DT_CODE[out.dtype], M, self.N, self.K, _ptr(ws),
                                  ws.numel(), stream_ptr(stream)))
        return out.reshape(*x.shape[:-1], self.N)

    __call__ = forward


def _make_ref_name(qname, tname, qtype, dt):
    def fn(inp, out, numel, stream=None):
        _need_cuda(inp, out)
        getattr(lib, f"dequantize_block_{qname}_{tname}")(_ptr(inp), _ptr(out), numel,
                                                           stream_ptr(stream))
        check()
        return out
    fn.__name__ = f"dequantize_block_{qname}_{tname}"
    fn.__doc__ = (f"Reference-named {qname} dequant to {tname}: (inp uint8 SoA, out, numel); "
                  "kernels/quant.cpp:257-268,477-488.")
    return fn


for _qn, _qt in (("q8_0", Q8_0), ("q4_k", Q4_K), ("q4_0", Q4_0)):
    for _tn, _dt in (("f16", F16), ("bf16", BF16), ("f32", F32)):
        globals()[f"dequantize_block_{_qn}_{_tn}"] = _make_ref_name(_qn, _tn, _qt, _dt)
