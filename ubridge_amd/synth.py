"""Seeded synthetic inputs shaped like the benchmark configurations.

numpy (PCG64) on the host for parity tests, so the CPU oracle and the GPU
see the same bytes.  Distributions follow the north-star configs: fp16 block
scales ~ U(0.001, 0.02), 4-bit codes uniform 0..15, int8 codes uniform
-127..127, Q4_K bytes random, activations N(0, 1).
"""
import numpy as np

Q4_0, Q8_0, Q4_K = 2, 8, 12


def rng(seed, stream=0):
    return np.random.Generator(np.random.PCG64([seed, stream]))


def _f16_scales(g, n, lo=0.001, hi=0.02):
    return g.uniform(lo, hi, n).astype(np.float16).view(np.uint16)


def make_weight_soa(qtype, N, K, seed, stream=1):
    """SoA bytes of a [N, K] weight in the reference layout."""
    g = rng(seed, stream)
    if qtype == Q4_0:
        nb = N * K // 32
        return np.concatenate([_f16_scales(g, nb).view(np.uint8),
                               g.integers(0, 256, nb * 16, dtype=np.uint8)])
    if qtype == Q8_0:
        nb = N * K // 32
        q = g.integers(-127, 128, nb * 32, dtype=np.int8)
        return np.concatenate([_f16_scales(g, nb).view(np.uint8), q.view(np.uint8)])
    if qtype == Q4_K:
        nb = N * K // 256
        hdr = np.empty((nb, 16), np.uint8)
        hdr[:, 0:2] = _f16_scales(g, nb).view(np.uint8).reshape(nb, 2)
        hdr[:, 2:4] = _f16_scales(g, nb).view(np.uint8).reshape(nb, 2)
        hdr[:, 4:16] = g.integers(0, 256, (nb, 12), dtype=np.uint8)
        return np.concatenate([hdr.ravel(), g.integers(0, 256, nb * 128, dtype=np.uint8)])
    raise ValueError(qtype)


def make_activations(M, K, seed, stream=2):
    return rng(seed, stream).standard_normal((M, K)).astype(np.float32)


def f32_to_bf16_bits(x):
    """Round-to-nearest-even f32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_bits_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def make_gptq_w4(K, N, group, seed, stream=3):
    """GPTQ-style int4 weight as the W4A16 config names it: qweight int32
    [K/8, N] (8 K-consecutive nibbles), bf16 scales ~ U(0.002, 0.02) [K/g, N],
    int4 zero-points ~ U{0..15} packed int32 [K/g, N/8]."""
    g = rng(seed, stream)
    qw = g.integers(0, 2**32, (K // 8, N), dtype=np.uint64).astype(np.uint32).view(np.int32)
    ng = (K + group - 1) // group
    scales = f32_to_bf16_bits(g.uniform(0.002, 0.02, (ng, N)).astype(np.float32))
    qz = g.integers(0, 2**32, (ng, N // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)
    return qw, scales, qz


def bf16_activations(M, K, seed, stream=4):
    return f32_to_bf16_bits(rng(seed, stream).standard_normal((M, K)).astype(np.float32))
