"""ctypes front of the CPU oracle (liboracle.so, built from ubridge_oracle.c).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use it as the checker.  The product path never imports it.
Arrays are numpy; bf16/f16 travel as uint16 bit patterns.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liboracle.so")

F32, F16, BF16 = 0, 1, 2
Q4_0, Q8_0, Q4_K = 2, 8, 12
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        _lib = ctypes.CDLL(_SO)
        _lib.orc_f16_to_f32.restype = ctypes.c_float
        _lib.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.orc_f32_to_f16.restype = ctypes.c_uint16
        _lib.orc_f32_to_f16.argtypes = [ctypes.c_float]
        _lib.orc_bf16_to_f32.restype = ctypes.c_float
        _lib.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.orc_f32_to_bf16.restype = ctypes.c_uint16
        _lib.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        _lib.orc_e4m3_to_f32.restype = ctypes.c_float
        _lib.orc_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        _lib.orc_f32_to_e4m3.restype = ctypes.c_uint8
        _lib.orc_f32_to_e4m3.argtypes = [ctypes.c_float]
        _lib.orc_moe_align_block_size.restype = ctypes.c_int
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


_OUT_NP = {F32: np.float32, F16: np.uint16, BF16: np.uint16}


def f32_to_bf16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_n(_p(x), _p(out), ctypes.c_size_t(x.size))
    return out


def bf16_to_f32(x):
    x = np.ascontiguousarray(x, dtype=np.uint16)
    out = np.empty(x.shape, np.float32)
    lib().orc_bf16_to_f32_n(_p(x), _p(out), ctypes.c_size_t(x.size))
    return out


def f32_to_f16_scalar(v):
    return lib().orc_f32_to_f16(float(v))


def f16_to_f32_scalar(h):
    return lib().orc_f16_to_f32(int(h))


def e4m3_to_f32(v):
    return lib().orc_e4m3_to_f32(int(v))


def f32_to_e4m3(v):
    return lib().orc_f32_to_e4m3(float(v))


def dequant(qtype, soa, numel, dtype):
    soa = np.ascontiguousarray(soa, dtype=np.uint8)
    out = np.empty(numel, _OUT_NP[dtype])
    fn = {Q8_0: lib().orc_dequant_q8_0, Q4_0: lib().orc_dequant_q4_0,
          Q4_K: lib().orc_dequant_q4_k}[qtype]
    fn(_p(soa), _p(out), ctypes.c_size_t(numel), ctypes.c_int(dtype))
    return out


def aos_to_soa(qtype, aos, nblocks):
    aos = np.ascontiguousarray(aos, dtype=np.uint8)
    out = np.empty_like(aos)
    lib().orc_aos_to_soa(qtype, _p(aos), _p(out), ctypes.c_size_t(nblocks))
    return out


def soa_to_aos(qtype, soa, nblocks):
    soa = np.ascontiguousarray(soa, dtype=np.uint8)
    out = np.empty_like(soa)
    lib().orc_soa_to_aos(qtype, _p(soa), _p(out), ctypes.c_size_t(nblocks))
    return out


def quantize_q8_0(x):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(x.size // 32 * 34, np.uint8)
    lib().orc_quantize_q8_0(_p(x), ctypes.c_size_t(x.size), _p(out))
    return out


def quantize_q8_k(x):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    nb = x.size // 256
    d = np.empty(nb, np.float32)
    qs = np.empty(x.size, np.int8)
    bs = np.empty(nb * 16, np.int16)
    lib().orc_quantize_q8_k(_p(x), ctypes.c_size_t(x.size), _p(d), _p(qs), _p(bs))
    return d, qs, bs


def qmatmul(qtype, w_soa, x, N, K, nthreads=1):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    M = x.shape[0]
    y = np.empty((M, N), np.float32)
    w_soa = np.ascontiguousarray(w_soa, dtype=np.uint8)
    lib().orc_qmatmul(qtype, _p(w_soa), _p(x), _p(y), M, N, K, nthreads)
    return y


def w8a16_gemm(a_bf16, w_i8, scales_bf16, M, K, N, group, rhs_t):
    out = np.empty((M, N), np.uint16)
    lib().orc_w8a16_gemm(_p(np.ascontiguousarray(a_bf16)), _p(np.ascontiguousarray(w_i8)),
                         _p(np.ascontiguousarray(scales_bf16)), _p(out), M, K, N, group, rhs_t)
    return out


def w4a16_dequant(qw, scales, qz, K, N, group):
    out = np.empty((K, N), np.uint16)
    lib().orc_w4a16_dequant(_p(np.ascontiguousarray(qw)), _p(np.ascontiguousarray(scales)),
                            _p(np.ascontiguousarray(qz)), _p(out), K, N, group)
    return out


def w4a16_gemm(a, qw, scales, qz, M, K, N, group, nthreads=1):
    out = np.empty((M, N), np.uint16)
    lib().orc_w4a16_gemm(_p(np.ascontiguousarray(a)), _p(np.ascontiguousarray(qw)),
                         _p(np.ascontiguousarray(scales)), _p(np.ascontiguousarray(qz)),
                         _p(out), M, K, N, group, nthreads)
    return out


def dequant_u4_ref(rhs, scale, zeros, K, N, group, dtype):
    out = np.empty((2 * K, N), np.uint16)
    lib().orc_dequant_u4_ref(_p(np.ascontiguousarray(rhs)), _p(np.ascontiguousarray(scale)),
                             _p(np.ascontiguousarray(zeros)), _p(out), K, N, group, dtype)
    return out


def fp8_quantize_rows(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    R, C = x.shape
    q = np.empty((R, C), np.uint8)
    s = np.empty(R, np.float32)
    lib().orc_fp8_quantize_rows(_p(x), _p(q), _p(s), R, C)
    return q, s


def fp8_gemm(a, sa, w, sw, M, K, N, nthreads=1):
    out = np.empty((M, N), np.uint16)
    lib().orc_fp8_gemm(_p(np.ascontiguousarray(a)), _p(np.ascontiguousarray(sa, np.float32)),
                       _p(np.ascontiguousarray(w)), _p(np.ascontiguousarray(sw, np.float32)),
                       _p(out), M, K, N, nthreads)
    return out


def topk_softmax(logits, k, norm, dtype):
    logits = np.ascontiguousarray(logits)
    T, E = logits.shape
    out = np.zeros((T, k), _OUT_NP[dtype])
    idx = np.zeros((T, k), np.int32)
    lib().orc_topk_softmax(_p(logits), _p(out), _p(idx), T, E, k, int(norm), dtype)
    return out, idx


def moe_align_block_size(topk_ids, E, bs, real_token_num=None, expert_map=None):
    topk_ids = np.ascontiguousarray(topk_ids, dtype=np.int32)
    T, k = topk_ids.shape
    max_padded = T * k + E * (bs - 1)
    sorted_ids = np.empty(max_padded, np.int32)
    experts = np.empty(max_padded // bs, np.int32)
    ntpp = np.zeros(1, np.int32)
    rt = None if real_token_num is None else np.array([real_token_num], np.int32)
    em = None if expert_map is None else np.ascontiguousarray(expert_map, dtype=np.int32)
    r = lib().orc_moe_align_block_size(_p(sorted_ids), _p(experts), _p(ntpp), _p(topk_ids),
                                       _p(rt), _p(em), E, bs, T, k)
    if r < 0:
        raise ValueError("moe_align_block_size: index out of range")
    return sorted_ids, experts, ntpp


def fused_moe(A, B, Bq, Bscale, bias, topk_w, sorted_ids, experts_ids, ntpp, M, K, N, E,
              topk_ids_size, top_k, bs, mul_routed_weight, C=None, nthreads=1):
    if C is None:
        C = np.zeros((topk_ids_size, N), np.uint16)
    lib().orc_fused_moe(_p(C), _p(A), _p(B), _p(Bq), _p(Bscale), _p(bias),
                        _p(None if topk_w is None else np.ascontiguousarray(topk_w, np.float32)),
                        _p(sorted_ids), _p(experts_ids), _p(ntpp), M, K, N, E, topk_ids_size,
                        top_k, bs, int(mul_routed_weight), int(bias is not None), nthreads)
    return C


def moe_combine(dt, y, e_out, w, idx, top, N, K, M, topk):
    """moe_{f16,bf16} (moe_host.cpp:27-93) on uint16 bit patterns; returns
    the combined copy of y."""
    y = np.array(y, np.uint16, copy=True)
    lib().orc_moe_combine(dt, _p(y), _p(np.ascontiguousarray(e_out, np.uint16)),
                          _p(np.ascontiguousarray(w, np.float32)),
                          _p(np.ascontiguousarray(idx, np.uint32)),
                          _p(np.ascontiguousarray(top, np.uint32)), N, K, M, topk)
    return y


def indexed_moe(dt, inp, w, out, idx, N, K, M, batch, topk, E):
    """indexed_moe_{f16,bf16} (moe_host.cpp:118-293) on uint16 bit patterns;
    `out` rows of pairs with an expert id >= E keep their contents."""
    out = np.array(out, np.uint16, copy=True)
    lib().orc_indexed_moe(dt, _p(np.ascontiguousarray(inp, np.uint16)),
                          _p(np.ascontiguousarray(w, np.uint16)), _p(out),
                          _p(np.ascontiguousarray(idx, np.uint32)), N, K, M, batch, topk, E)
    return out
