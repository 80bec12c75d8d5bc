"""Host-side mirror of Ubridge's MoE operators (src/ffi.rs:44-236):

  topk_softmax_{f32,f16,bf16}   kernels/topk_softmax_host.cpp:178-208
  moe_align_block_size          kernels/moe_align_host.cpp:923-935
  invoke_fused_moe_{f16,bf16}   kernels/fused_moe_host.cpp:504-536
  moe_{f16,bf16}, indexed_moe_{f16,bf16}   kernels/moe_host.cpp (legacy)
  topsaten_{topk_softmax_f32, moe_align_block_size, fused_moe_gemm}
                                kernels/topsaten_moe_wrapper.cpp:80-216
                                (status-returning, src/ffi.rs:671-715)

plus the W8A16 expert GEMM, silu_and_mul and the top-k combine, and
`fused_moe`, which chains them in the order a vLLM-style MoE layer calls the
reference (router softmax -> align -> gate/up GEMM -> SiLU*up -> down GEMM
with routed weights -> sum over the k slots).  All compute is in
libubridge_hip.so; torch only provides device buffers and the stream.
"""
import ctypes

import torch

from ._lib import check, lib, register
from .ops import _DT_CODE, _DT_NAME, _need_cuda, _ptr, stream_ptr

_vp, _i, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
for _t in ("f32", "f16", "bf16"):
    register(f"topk_softmax_{_t}", None, [_vp, _vp, _vp, _i, _i, _i, _i, _vp])
register("moe_align_block_size", None, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp])
for _t in ("f16", "bf16"):
    register(f"invoke_fused_moe_{_t}", None,
             [_vp] * 8 + [_i] * 9 + [_vp])
    register(f"moe_{_t}", None, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp])
    register(f"indexed_moe_{_t}", None, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp])
register("ubridge_fused_moe_w8a16", _i, [_vp] * 9 + [_i] * 10 + [_vp])
register("ubridge_fused_moe_w8a16_silu", _i, [_vp] * 8 + [_i] * 9 + [_vp])
register("ubridge_fused_moe_w8a16_combine", _i, [_vp] * 10 + [_i] * 10 + [_vp])
register("ubridge_silu_and_mul", _i, [_vp, _vp, _i, _i, _i, _vp])
register("ubridge_moe_route", _i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp])
register("ubridge_moe_sum", _i, [_vp, _vp, _i, _i, _i, _i, _vp])
register("ubridge_device_error", _i, [_vp])
register("topsaten_topk_softmax_f32", _i, [_vp] * 4 + [_i] * 4 + [_vp])
register("topsaten_moe_align_block_size", _i, [_vp] * 4 + [_i] * 4 + [_vp])
register("topsaten_fused_moe_gemm", _i, [_vp] * 8 + [_i] * 8 + [_vp])
register("topsaten_release_graph_workspace_pool", None, [_vp])


def device_error(stream=None):
    """Synchronize the stream and raise if a kernel flagged an out-of-range
    index (the reference traps on the device instead)."""
    check(lib.ubridge_device_error(stream_ptr(stream)))


def topk_softmax(gating, topk, renormalize=True, stream=None):
    """gating [T, E] (f32/f16/bf16) -> (weights [T, topk] same dtype, ids int32)."""
    _need_cuda(gating)
    gating = gating.contiguous()
    T, E = gating.shape
    w = torch.empty(T, topk, dtype=gating.dtype, device=gating.device)
    ids = torch.empty(T, topk, dtype=torch.int32, device=gating.device)
    getattr(lib, f"topk_softmax_{_DT_NAME[gating.dtype]}")(
        _ptr(gating), _ptr(w), _ptr(ids), T, E, topk, int(renormalize), stream_ptr(stream))
    check()
    return w, ids


def moe_align_block_size(topk_ids, num_experts, block_size, real_token_num=None, expert_map=None,
                         stream=None):
    """topk_ids int32 [T, k] -> (sorted_ids, experts_ids, num_tokens_post_pad),
    buffers sized T*k + E*(bs-1) and that / bs, as the reference's caller
    allocates them."""
    _need_cuda(topk_ids)
    topk_ids = topk_ids.contiguous()
    T, k = topk_ids.shape
    max_padded = T * k + num_experts * (block_size - 1)
    dev = topk_ids.device
    sorted_ids = torch.empty(max_padded, dtype=torch.int32, device=dev)
    experts = torch.empty(max_padded // block_size, dtype=torch.int32, device=dev)
    ntpp = torch.empty(1, dtype=torch.int32, device=dev)
    rt = None
    if real_token_num is not None:
        rt = real_token_num if torch.is_tensor(real_token_num) else torch.tensor(
            [real_token_num], dtype=torch.int32, device=dev)
    lib.moe_align_block_size(_ptr(sorted_ids), _ptr(experts), _ptr(ntpp), _ptr(topk_ids), _ptr(rt),
                             _ptr(expert_map), num_experts, block_size, T, k, stream_ptr(stream))
    check()
    return sorted_ids, experts, ntpp


def moe_route(gating, topk, num_experts, block_size, renormalize=True, stream=None):
    """topk_softmax + moe_align_block_size in one call.  Returns (weights T [T, k], weights f32 [T, k], ids,
    sorted_ids, experts_ids, num_tokens_post_pad), the same values as the two
    reference-named operators."""
    _need_cuda(gating)
    gating = gating.contiguous()
    T, E = gating.shape
    dev = gating.device
    w = torch.empty(T, topk, dtype=gating.dtype, device=dev)
    wf = torch.empty(T, topk, dtype=torch.float32, device=dev)
    ids = torch.empty(T, topk, dtype=torch.int32, device=dev)
    max_padded = T * topk + num_experts * (block_size - 1)
    sorted_ids = torch.empty(max_padded, dtype=torch.int32, device=dev)
    experts = torch.empty(max_padded // block_size, dtype=torch.int32, device=dev)
    ntpp = torch.empty(1, dtype=torch.int32, device=dev)
    check(lib.ubridge_moe_route(_ptr(gating), _DT_CODE[gating.dtype], _ptr(w), _ptr(wf), _ptr(ids),
                                _ptr(sorted_ids), _ptr(experts), _ptr(ntpp), T, E, topk,
                                int(renormalize), block_size, stream_ptr(stream)))
    return w, wf, ids, sorted_ids, experts, ntpp


def topsaten_topk_softmax(gating, topk, norm_topk_prob=True, stream=None):
    """The status-returning top-k (topsaten_moe_wrapper.cpp:80-101): gating f32
    [T, E] -> (weights f32 [T, k], ids int32, token_expert_indices int32 with
    [t, j] = j * T + t)."""
    _need_cuda(gating)
    gating = gating.float().contiguous()
    T, E = gating.shape
    dev = gating.device
    w = torch.empty(T, topk, dtype=torch.float32, device=dev)
    ids = torch.empty(T, topk, dtype=torch.int32, device=dev)
    tei = torch.empty(T, topk, dtype=torch.int32, device=dev)
    check(lib.topsaten_topk_softmax_f32(_ptr(gating), _ptr(w), _ptr(ids), _ptr(tei), T, E, topk,
                                        int(norm_topk_prob), stream_ptr(stream)))
    return w, ids, tei


def topsaten_moe_align_block_size(topk_ids, num_experts, block_size, stream=None):
    """The status-returning align (topsaten_moe_wrapper.cpp:108-141); buffers
    as moe_align_block_size sizes them."""
    _need_cuda(topk_ids)
    topk_ids = topk_ids.contiguous()
    T, k = topk_ids.shape
    max_padded = T * k + num_experts * (block_size - 1)
    dev = topk_ids.device
    sorted_ids = torch.empty(max_padded, dtype=torch.int32, device=dev)
    experts = torch.empty(max_padded // block_size, dtype=torch.int32, device=dev)
    ntpp = torch.empty(1, dtype=torch.int32, device=dev)
    check(lib.topsaten_moe_align_block_size(_ptr(sorted_ids), _ptr(experts), _ptr(ntpp),
                                            _ptr(topk_ids), T, k, num_experts, block_size,
                                            stream_ptr(stream)))
    return sorted_ids, experts, ntpp


_TOPSATEN_DT = {torch.float16: 4, torch.bfloat16: 5, torch.float32: 8}


def topsaten_fused_moe_gemm(A, B, topk_weights, topk_ids, sorted_ids, experts_ids, ntpp,
                            mul_routed_weight, block_size, C=None, stream=None):
    """The status-returning grouped GEMM (topsaten_moe_wrapper.cpp:152-208):
    A [T, hidden], B [E, inter, hidden] -> C [T, k, inter]."""
    _need_cuda(A, B, sorted_ids, experts_ids, ntpp)
    T, hidden = A.shape
    E, inter, _ = B.shape
    k = topk_ids.shape[1]
    if C is None:
        C = torch.empty(T, k, inter, dtype=A.dtype, device=A.device)
    tw = None if topk_weights is None else topk_weights.float().contiguous()
    check(lib.topsaten_fused_moe_gemm(_ptr(C), _ptr(A), _ptr(B), _ptr(tw), _ptr(topk_ids),
                                      _ptr(sorted_ids), _ptr(experts_ids), _ptr(ntpp),
                                      int(mul_routed_weight), k, block_size, T, hidden, inter, E,
                                      _TOPSATEN_DT[A.dtype], stream_ptr(stream)))
    return C


def invoke_fused_moe(A, B, C, topk_weights, sorted_ids, experts_ids, ntpp, top_k, block_size,
                     mul_routed_weight, B_scale=None, bias=None, topk_ids_size=None, stream=None):
    """Grouped expert GEMM over the sorted blocks (fused_moe_host.cpp:43-252).
    B: [E, N, K] in A's dtype (invoke_fused_moe_*) or int8 with per-channel
    B_scale [E, N] (W8A16).  C: [topk_ids_size, N]."""
    _need_cuda(A, B, C, sorted_ids, experts_ids, ntpp)
    E, N, K = B.shape
    M = A.shape[0]
    tis = topk_ids_size if topk_ids_size is not None else C.shape[0]
    tw = None if topk_weights is None else topk_weights.float().contiguous()
    args = (_ptr(C), _ptr(A), _ptr(B))
    tail = (_ptr(tw), _ptr(sorted_ids), _ptr(experts_ids), _ptr(ntpp), M, K, N, E, tis, top_k,
            block_size, int(mul_routed_weight), int(bias is not None))
    if B.dtype == torch.int8:
        check(lib.ubridge_fused_moe_w8a16(*args, _ptr(B_scale), _ptr(bias), *tail,
                                          _DT_CODE[A.dtype], stream_ptr(stream)))
    else:
        getattr(lib, f"invoke_fused_moe_{_DT_NAME[A.dtype]}")(*args, _ptr(bias), *tail,
                                                             stream_ptr(stream))
        check()
    return C


def fused_moe_down_combine(A, B, B_scale, topk_weights, sorted_ids, experts_ids, ntpp, top_k,
                           block_size, C=None, out=None, mul_routed_weight=True, bias=None,
                           topk_ids_size=None, stream=None):
    """Down W8A16 expert GEMM and the top-k combine in one call: C
    [topk_ids_size, N] as invoke_fused_moe writes it and out [T, N] = the
    slot-order sum of each token's top_k rows (moe_sum's bits)."""
    _need_cuda(A, B, B_scale, sorted_ids, experts_ids, ntpp)
    E, N, K = B.shape
    tis = topk_ids_size if topk_ids_size is not None else (C.shape[0] if C is not None
                                                            else A.shape[0])
    T = tis // top_k
    if C is None:
        C = torch.empty(tis, N, dtype=A.dtype, device=A.device)
    if out is None:
        out = torch.empty(T, N, dtype=A.dtype, device=A.device)
    tw = None if topk_weights is None else topk_weights.float().contiguous()
    check(lib.ubridge_fused_moe_w8a16_combine(
        _ptr(out), _ptr(C), _ptr(A), _ptr(B), _ptr(B_scale), _ptr(bias), _ptr(tw),
        _ptr(sorted_ids), _ptr(experts_ids), _ptr(ntpp), A.shape[0], K, N, E,
        tis, top_k, block_size, int(mul_routed_weight), int(bias is not None),
        _DT_CODE[A.dtype], stream_ptr(stream)))
    return out


def fused_moe_gate_up_silu(A, B, B_scale, sorted_ids, experts_ids, ntpp, top_k, block_size,
                           bias=None, out=None, topk_ids_size=None, stream=None):
    """Gate/up W8A16 expert GEMM with silu_and_mul fused into its epilogue:
    B int8 [E, 2I, K] (gate rows, then up rows) -> [topk_ids_size, I], the
    same values as invoke_fused_moe followed by silu_and_mul."""
    _need_cuda(A, B, B_scale, sorted_ids, experts_ids, ntpp)
    E, N, K = B.shape
    tis = topk_ids_size if topk_ids_size is not None else A.shape[0] * top_k
    if out is None:
        out = torch.empty(tis, N // 2, dtype=A.dtype, device=A.device)
    check(lib.ubridge_fused_moe_w8a16_silu(_ptr(out), _ptr(A), _ptr(B), _ptr(B_scale), _ptr(bias),
                                           _ptr(sorted_ids), _ptr(experts_ids), _ptr(ntpp),
                                           A.shape[0], K, N, E, tis, top_k, block_size,
                                           int(bias is not None), _DT_CODE[A.dtype],
                                           stream_ptr(stream)))
    return out


def silu_and_mul(x, out=None, stream=None):
    """x [T, 2d] -> silu(x[:, :d]) * x[:, d:]."""
    _need_cuda(x)
    T, d2 = x.shape
    if out is None:
        out = torch.empty(T, d2 // 2, dtype=x.dtype, device=x.device)
    check(lib.ubridge_silu_and_mul(_ptr(out), _ptr(x.contiguous()), T, d2 // 2, _DT_CODE[x.dtype],
                                   stream_ptr(stream)))
    return out


def moe_sum(x, T, k, out=None, stream=None):
    """x [T*k, N] -> sum over the k slots of each token -> [T, N]."""
    _need_cuda(x)
    N = x.shape[-1]
    if out is None:
        out = torch.empty(T, N, dtype=x.dtype, device=x.device)
    check(lib.ubridge_moe_sum(_ptr(out), _ptr(x.contiguous()), T, k, N, _DT_CODE[x.dtype],
                              stream_ptr(stream)))
    return out


def moe_combine(y, e_out, w, idx, top, topk, stream=None):
    """Legacy moe_{f16,bf16}: y[idx[k]] += e_out[k] * w[idx[k]*topk + top[k]] (in place)."""
    _need_cuda(y, e_out, w, idx, top)
    N, M = y.shape
    K = idx.numel()
    getattr(lib, f"moe_{_DT_NAME[y.dtype]}")(_ptr(y), _ptr(e_out), _ptr(w), _ptr(idx), _ptr(top),
                                             N, K, M, topk, stream_ptr(stream))
    check()
    return y


def indexed_moe(x, w, idx, out=None, stream=None):
    """Legacy indexed_moe_{f16,bf16}: x [B, M, K] (M == 1 or topk), w [E, N, K],
    idx [B, topk] -> out [B, topk, N] = w[idx] . x (row i reads x[b, 0] when
    M == 1, else x[b, i]).  Rows whose expert id is >= E keep the contents
    of `out` (zeros when it is not given)."""
    _need_cuda(x, w, idx)
    B, M, K = x.shape
    E, N, _ = w.shape
    topk = idx.shape[1]
    if out is None:
        out = torch.zeros(B, topk, N, dtype=x.dtype, device=x.device)
    getattr(lib, f"indexed_moe_{_DT_NAME[x.dtype]}")(_ptr(x.contiguous()), _ptr(w), _ptr(out),
                                                     _ptr(idx), N, K, M, B, topk, E,
                                                     stream_ptr(stream))
    check()
    return out


class FusedMoE:
    """A W8A16 (or bf16) MoE layer driven through the reference call order.

    w13: [E, 2I, H] gate/up experts (int8 with per-channel scales s13 [E, 2I],
    or bf16), w2: [E, H, I] down experts (int8 + s2 [E, H], or bf16).
    """

    def __init__(self, w13, w2, s13=None, s2=None, topk=8, renormalize=True, block_size=32):
        self.w13, self.w2, self.s13, self.s2 = w13, w2, s13, s2
        self.topk, self.renormalize, self.block_size = topk, renormalize, block_size
        self.E = w13.shape[0]

    def forward(self, x, router_logits, stream=None):
        T, H = x.shape
        k, E, bs = self.topk, self.E, self.block_size
        _, wf, ids, sorted_ids, experts, ntpp = moe_route(router_logits, k, E, bs,
                                                          self.renormalize, stream=stream)
        if self.w13.dtype == torch.int8:  # gate/up GEMM and silu_and_mul in one kernel
            act = fused_moe_gate_up_silu(x, self.w13, self.s13, sorted_ids, experts, ntpp, k, bs,
                                         stream=stream)
        else:
            I2 = self.w13.shape[1]
            h1 = torch.empty(T * k, I2, dtype=x.dtype, device=x.device)
            invoke_fused_moe(x, self.w13, h1, None, sorted_ids, experts, ntpp, k, bs, False,
                             stream=stream)
            act = silu_and_mul(h1, stream=stream)
        h2 = torch.empty(T * k, H, dtype=x.dtype, device=x.device)
        if self.w2.dtype == torch.int8:  # down GEMM and the top-k combine in one call
            return fused_moe_down_combine(act, self.w2, self.s2, wf.reshape(-1), sorted_ids,
                                          experts, ntpp, k, bs, C=h2, stream=stream)
        invoke_fused_moe(act, self.w2, h2, wf.reshape(-1), sorted_ids, experts, ntpp, k,
                         bs, True, B_scale=self.s2, stream=stream)
        return moe_sum(h2, T, k, stream=stream)

    __call__ = forward
