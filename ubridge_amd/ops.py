"""Host-side mirror of Ubridge's quantized-matmul operator interface.

Every function here is a thin torch-facing wrapper over one C-ABI entry point
of libubridge_hip.so (include/ubridge_hip.h).  torch only supplies device
memory and the current HIP stream; all arithmetic runs in the HIP kernels.
Names and argument meanings follow the reference's operators:
  dequantize_block_{q8_0,q4_k}_{f16,bf16,f32}  kernels/quant.cpp:257-268,477-488
  quantize_block_q8_0_{bf16,f16,f32}           kernels/quant.cpp:331-353
  QMatMul (Candle's quantized matmul), served on the reference by dequant +
  matmul_bf16 (kernels/matmul.cpp:1143-1184), here by the fused GEMV (decode
  sizes) or, from 64 tokens (Q4_K; 40 for Q4_0 / Q8_0), by that same sequence
  on slabs (dequantize, then a hipBLASLt GEMM).
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


# --------------------------------------------------------- quantized GEMMs
def w4a16_gemm(a, qweight, scales, qzeros, group_size=128, out=None, stream=None):
    """out[M,N] = a[M,K] @ deq(W)[K,N] for GPTQ-style int4 weights:
    qweight int32 [K/8, N], scales bf16/f16 [K/g, N], qzeros int32 [K/g, N/8]."""
    _need_cuda(a, qweight, scales, qzeros)
    a = a.contiguous()
    M, K = a.shape
    N = qweight.shape[1]
    if out is None:
        out = torch.empty(M, N, dtype=a.dtype, device=a.device)
    check(lib.ubridge_w4a16_gemm(_ptr(a), _ptr(qweight), _ptr(scales), _ptr(qzeros), _ptr(out),
                                 M, K, N, group_size, _DT_CODE[a.dtype], stream_ptr(stream)))
    return out


def gemm_dense(a, w, w_transposed=False, out=None, stream=None):
    """out = a @ w (w [K,N]) or a @ w.T (w [N,K], w_transposed=True)."""
    _need_cuda(a, w)
    a = a.contiguous()
    M, K = a.shape
    N = w.shape[0] if w_transposed else w.shape[1]
    if out is None:
        out = torch.empty(M, N, dtype=a.dtype, device=a.device)
    check(lib.ubridge_gemm_dense(_ptr(a), _ptr(w.contiguous()), _ptr(out), M, K, N,
                                 int(w_transposed), _DT_CODE[a.dtype], stream_ptr(stream)))
    return out


_I, _F = ctypes.c_int32, ctypes.c_float


class GemmOpParas(ctypes.Structure):
    """GEMM_OP_PARAS (src/gemm_tuner.rs:222-258), as UbridgeGemmOpParas."""
    _fields_ = [(n, _I) for n in (
        "input_dtype", "output_dtype", "csb_batch", "sip_batch", "lhs_csb_k", "rhs_csb_k",
        "lhs_csb_m", "rhs_csb_n", "sip_m", "sip_k", "sip_n", "batch_multicore", "lhs_multicore",
        "rhs_multicore", "lhs_pingpong", "rhs_pingpong", "sdma_lhs_pingpong", "sdma_rhs_pingpong",
        "rhs_repeat_copy", "lhs_transpose", "rhs_transpose", "out_transpose")] + \
        [(n, _F) for n in ("alpha", "beta", "addmm_beta", "coef", "act_mode")] + \
        [(n, _I) for n in ("bias", "act_en", "input_batch", "input_m", "input_k", "input_n")]


_REF_DATATYPE = {torch.float16: 4, torch.bfloat16: 5, "i8": 0, "i4": 15}
lib.ubridge_get_gemm_launch_params.restype = ctypes.POINTER(GemmOpParas)
lib.ubridge_get_gemm_launch_params.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_size_t,
                                               ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
                                               ctypes.c_int]


def get_gemm_launch_params(dtype, weight_type, b, m, k, n, rhs_trans):
    """GcuDevice::get_gemm_launch_params (src/gcu_device.rs:185-198): the
    cached launch parameters for a GEMM shape.  dtype is the activation
    torch dtype; weight_type the same dtype (dense), "i8" or "i4"."""
    p = lib.ubridge_get_gemm_launch_params(_REF_DATATYPE[dtype], _REF_DATATYPE[weight_type], b, m,
                                           k, n, int(rhs_trans))
    if not p:
        check()
    return p.contents


def _ref_mm_args(dtype, batch, m, k, n, rhs_t, broadcast, wtype):
    # input_dtype, batch, m, k, n, lhs/rhs/batch multicore, lhs_t, rhs_t,
    # alpha, beta, addmm_beta, sip_m, sip_k, sip_n, broadcasted_weight -- the
    # tiling fields from get_gemm_launch_params, as the reference's caller
    # passes them (gcu_device.rs:185-198 then matmul_*)
    p = get_gemm_launch_params(dtype, wtype, batch, m, k, n, rhs_t)
    return [_DT_CODE[dtype], batch, m, k, n, p.lhs_multicore, p.rhs_multicore, p.batch_multicore,
            0, int(rhs_t), 1.0, 0.0, 0.0, p.sip_m, p.sip_k, p.sip_n, int(broadcast)]


def matmul_quant(a, w, scales, zeros=None, bits=8, group_size=-1, rhs_transpose=False, out=None,
                 stream=None):
    """Reference matmul_{bf16,f16}_{4bit,8bit} (kernels/matmul.cpp:1186-1215).
    a [B?, M, K]; 8-bit w int8 [K, N] ([N, K] if rhs_transpose); 4-bit w uint8
    [K/2, N] (low nibble = even k); scales (and 4-bit zeros) dtype [K/g, N]."""
    _need_cuda(a, w, scales)
    a = a.contiguous()
    a3 = a if a.dim() == 3 else a.unsqueeze(0)
    B, M, K = a3.shape
    N = (w.shape[0] if rhs_transpose else w.shape[1])
    if out is None:
        out = torch.empty(B, M, N, dtype=a.dtype, device=a.device)
    name = f"matmul_{_DT_NAME[a.dtype]}_{bits}bit"
    getattr(lib, name)(_ptr(a3), _ptr(w), _ptr(out), _ptr(scales), _ptr(zeros),
                       *_ref_mm_args(a.dtype, B, M, K, N, rhs_transpose, True,
                                     "i8" if bits == 8 else "i4"), group_size,
                       stream_ptr(stream))
    check()
    return out if a.dim() == 3 else out[0]


def matmul(a, b, rhs_transpose=False, out=None, stream=None):
    """Reference dense matmul_{bf16,f16} (kernels/matmul.cpp:1181-1184), batched."""
    _need_cuda(a, b)
    a3 = a.contiguous() if a.dim() == 3 else a.contiguous().unsqueeze(0)
    B, M, K = a3.shape
    N = b.shape[-2] if rhs_transpose else b.shape[-1]
    broadcast = b.dim() == 2
    if out is None:
        out = torch.empty(B, M, N, dtype=a.dtype, device=a.device)
    getattr(lib, f"matmul_{_DT_NAME[a.dtype]}")(_ptr(a3), _ptr(b.contiguous()), _ptr(out),
                                               *_ref_mm_args(a.dtype, B, M, K, N, rhs_transpose,
                                                             broadcast, a.dtype),
                                               stream_ptr(stream))
    check()
    return out if a.dim() == 3 else out[0]


def dequant_u4(rhs, scale, zeros, group_size=-1, out=None, stream=None):
    """Reference dequant_{bf16,f16} (kernels/dequant_host.cpp:298-307): rhs uint8
    [K, N] packs 2K rows; returns [2K, N] in scale's dtype."""
    _need_cuda(rhs, scale, zeros)
    K, N = rhs.shape
    if out is None:
        out = torch.empty(2 * K, N, dtype=scale.dtype, device=rhs.device)
    getattr(lib, f"dequant_{_DT_NAME[scale.dtype]}")(_ptr(out), _ptr(rhs), _ptr(scale), _ptr(zeros),
                                                     K, N, 0, group_size, stream_ptr(stream))
    check()
    return out


# ----------------------------------------------------------- launch knobs
TUNE_KNOBS = ("gemv_lds_rows", "gemv_lds_waves", "gemv_rows", "gemv_iters", "gemm_tile",
              "gemv_mfma_m", "w4a16_path", "moe_gemm_path",
              "gemv_mm")


def tune_set(name, value):
    """Override a launch-shape rule process-wide (0 restores the automatic
    choice); the host tiling choice of the reference's gemm_tuner.rs."""
    check(lib.ubridge_tune_set(name.encode(), int(value)))


def tune_get(name):
    v = lib.ubridge_tune_get(name.encode())
    check()
    return v


# --------------------------------------------------------- device scratch
# The scratch some routes need (K-split partials, dequantized weight slabs)
# comes from a caller-registered stream-ordered allocator, or else from the
# library's per-(device, stream) pool; see include/ubridge_hip.h.
_WS_ALLOC = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t,
                             ctypes.c_void_p, ctypes.c_void_p)
_WS_FREE = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p)
_lib.register("ubridge_set_workspace_allocator", ctypes.c_int,
              [_WS_ALLOC, _WS_FREE, ctypes.c_void_p])
_lib.register("ubridge_release_workspace", ctypes.c_int, [ctypes.c_void_p])
_lib.register("ubridge_init", ctypes.c_int, [])
_lib.register("ubridge_workspace_stats", ctypes.c_int,
              [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t),
               ctypes.POINTER(ctypes.c_long)])
_allocator_keep = []  # the registered callbacks must outlive their registration


class TorchWorkspaceAllocator:
    """Serves the library's scratch from torch's caching allocator on the
    call's stream: stream-ordered (a block handed back on a stream is reused
    only by work ordered after it there) and, inside torch.cuda.graph, drawn
    from the graph's private pool.  `live` counts blocks not yet handed
    back, `calls` allocations served."""

    def __init__(self, device=None):
        self.device = torch.cuda.current_device() if device is None else device
        self.live = {}
        self.calls = 0

        def _alloc(pp, nbytes, stream, _ctx):
            try:
                s = stream if stream else 0
                p = torch.cuda.caching_allocator_alloc(int(nbytes), self.device, s)
            except Exception:  # noqa: BLE001 -- reported to the library as failure
                return 1
            self.live[p] = int(nbytes)
            self.calls += 1
            pp[0] = p
            return 0

        def _free(p, _stream, _ctx):
            self.live.pop(p, None)
            torch.cuda.caching_allocator_delete(p)

        self._cb = (_WS_ALLOC(_alloc), _WS_FREE(_free))


def set_workspace_allocator(allocator):
    """Register a TorchWorkspaceAllocator (None: back to the library pool)."""
    if allocator is None:
        check(lib.ubridge_set_workspace_allocator(_WS_ALLOC(), _WS_FREE(), None))
        return
    _allocator_keep.append(allocator)
    check(lib.ubridge_set_workspace_allocator(allocator._cb[0], allocator._cb[1], None))


def init():
    """hipBLASLt set-up of the current device (the first eager call does it;
    needed first only when a process's first call is made inside a graph
    capture)."""
    check(lib.ubridge_init())


def release_workspace(stream=None):
    """Synchronize `stream` and free the library pool's buffers for it."""
    check(lib.ubridge_release_workspace(stream_ptr(stream)))


def workspace_stats():
    """(pool buffers live, their bytes, caller-allocator blocks outstanding)."""
    n, b, c = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_long()
    check(lib.ubridge_workspace_stats(ctypes.byref(n), ctypes.byref(b), ctypes.byref(c)))
    return n.value, b.value, c.value
