"""Write the golden fixtures in tests/golden/*.npz.

The reference holds no golden vectors for this path (its only numeric
harness, kernels/moe_host.cpp:379-525, is compiled out and unseeded), so the
fixtures come from this second, independent restatement of the published
formats, written in vectorised numpy rather than the C oracle's loops:

  * GGML block formats Q4_0 / Q8_0 / Q4_K (layouts: kernels/quant.cpp:64-185;
    the 6-bit scale unpacking: get_scale_min_k4, quant.cpp:356-363);
  * Candle's activation quantizers (BlockQ8_0 / BlockQ8K from_float) and its
    generic vec_dot (integer block sums scaled per block);
  * topk_softmax (topk_softmax_host.cpp:103-176) and moe_align_block_size
    (moe_align_host.cpp:587-921).

tests/test_oracle.py checks the C oracle against these files bit for bit
(integer and dequant outputs) or to float-summation-order tolerance.

    python tests/golden/make_golden.py
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f16_bits(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def f16_val(b):
    return np.asarray(b, np.uint16).view(np.float16).astype(np.float32)


def bf16_bits(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_val(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- formats
def q8_0_dequant(soa, nb):
    d = f16_val(soa[: 2 * nb].view(np.uint16))
    q = soa[2 * nb:].view(np.int8).reshape(nb, 32).astype(np.float32)
    f32 = (q * d[:, None]).ravel()
    f16 = f16_bits(f32)
    dbf = bf16_val(bf16_bits(d))
    bf = bf16_bits((q * dbf[:, None]).ravel())
    return f32, f16, bf


def q4_0_dequant(soa, nb):
    d = f16_val(soa[: 2 * nb].view(np.uint16))
    qs = soa[2 * nb:].reshape(nb, 16)
    q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.float32) - 8.0
    f32 = (q * d[:, None]).ravel()
    return f32, f16_bits(f32), bf16_bits(f32)


def q4_k_scales(sc12):
    """(nb,12) packed bytes -> (nb,8) scales, (nb,8) mins, 6-bit each."""
    s = sc12.astype(np.int32)
    sc = np.zeros((s.shape[0], 8), np.int32)
    mn = np.zeros_like(sc)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, mn


def q4_k_codes(qs128):
    """(nb,128) bytes -> (nb,256) codes in element order."""
    q = qs128.reshape(-1, 4, 32)
    return np.concatenate([q & 15, q >> 4], axis=2).reshape(-1, 256).astype(np.int32)


def q4_k_dequant(soa, nb):
    hdr = soa[: 16 * nb].reshape(nb, 16)
    d = f16_val(hdr[:, 0:2].copy().view(np.uint16).ravel())
    dmin = f16_val(hdr[:, 2:4].copy().view(np.uint16).ravel())
    sc, mn = q4_k_scales(hdr[:, 4:16])
    codes = q4_k_codes(soa[16 * nb:].reshape(nb, 128)).reshape(nb, 8, 32).astype(np.float32)
    dsc = (d[:, None] * sc.astype(np.float32))[:, :, None]
    mm = (dmin[:, None] * mn.astype(np.float32))[:, :, None]
    f32 = (dsc * codes - mm).astype(np.float32).ravel()
    return f32, f16_bits(f32), bf16_bits(f32)


# -------------------------------------------------------- activation quant
def round_half_away(v):
    t = np.trunc(v)
    return t + np.sign(v) * (np.abs(v - t) >= np.float32(0.5))


def quant_q8_0(x):
    xb = x.reshape(-1, 32).astype(np.float32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    v = (xb * idv[:, None]).astype(np.float32)
    q = round_half_away(v).astype(np.int8)
    return f16_bits(d), q


def quant_q8_k(x):
    xb = x.reshape(-1, 256).astype(np.float32)
    ia = np.argmax(np.abs(xb), axis=1)  # first index of the maximum
    mx = xb[np.arange(xb.shape[0]), ia]
    d = np.zeros(xb.shape[0], np.float32)
    q = np.zeros(xb.shape, np.int8)
    nz = mx != 0
    iscale = (np.float32(-128) / mx[nz]).astype(np.float32)
    v = (iscale[:, None] * xb[nz]).astype(np.float32)
    v = round_half_away(v)
    q[nz] = np.minimum(v, 127).astype(np.int8)
    d[nz] = (np.float32(1) / iscale).astype(np.float32)
    bs = q.reshape(-1, 16, 16).astype(np.int32).sum(axis=2).astype(np.int16)
    return d, q, bs


# ---------------------------------------------------------------- qmatmul
def qmatmul(qt, soa, x, N, K):
    """Candle method; block results summed in f64 (the C oracle sums in f32,
    so the fixture comparison uses a summation-order tolerance)."""
    M = x.shape[0]
    y = np.zeros((M, N), np.float64)
    if qt in (2, 8):
        nb = N * K // 32
        dw = f16_val(soa[: 2 * nb].view(np.uint16)).reshape(N, K // 32).astype(np.float64)
        if qt == 8:
            cw = soa[2 * nb:].view(np.int8).reshape(N, K // 32, 32).astype(np.int64)
        else:
            qs = soa[2 * nb:].reshape(N, K // 32, 16)
            cw = np.concatenate([qs & 15, qs >> 4], axis=2).astype(np.int64) - 8
        for m in range(M):
            dah, qa = quant_q8_0(x[m])
            da = f16_val(dah).astype(np.float64)
            isum = np.einsum("nbj,bj->nb", cw, qa.reshape(K // 32, 32).astype(np.int64))
            y[m] = (isum * dw * da[None, :]).sum(axis=1)
    else:
        nb = N * K // 256
        hdr = soa[: 16 * nb].reshape(nb, 16)
        d = f16_val(hdr[:, 0:2].copy().view(np.uint16).ravel()).astype(np.float64).reshape(N, -1)
        dmin = f16_val(hdr[:, 2:4].copy().view(np.uint16).ravel()).astype(np.float64).reshape(N, -1)
        sc, mn = q4_k_scales(hdr[:, 4:16])
        sc = sc.reshape(N, K // 256, 8).astype(np.int64)
        mn = mn.reshape(N, K // 256, 8).astype(np.int64)
        codes = q4_k_codes(soa[16 * nb:].reshape(nb, 128)).reshape(N, K // 256, 8, 32)
        for m in range(M):
            da, qa, bs = quant_q8_k(x[m])
            qa = qa.reshape(K // 256, 8, 32).astype(np.int64)
            sub = np.einsum("nbsj,bsj->nbs", codes.astype(np.int64), qa)
            isum = (sub * sc).sum(axis=2)
            bs32 = bs.reshape(K // 256, 8, 2).astype(np.int64).sum(axis=2)
            imin = (mn * bs32[None]).sum(axis=2)
            dd = da.astype(np.float64)[None, :]
            y[m] = (d * dd * isum - dmin * dd * imin).sum(axis=1)
    return y.astype(np.float32)


# ------------------------------------------------------------------- MoE
def topk_softmax(logits, k, norm):
    x = logits.astype(np.float32)
    p = np.exp((x - x.max(axis=1, keepdims=True)).astype(np.float64))
    p = p / p.sum(axis=1, keepdims=True)
    idx = np.argsort(-p, axis=1, kind="stable")[:, :k].astype(np.int32)
    w = np.take_along_axis(p, idx, axis=1)
    if norm:
        w = w / w.sum(axis=1, keepdims=True)
    return w.astype(np.float32), idx


def moe_align(topk_ids, E, bs):
    flat = topk_ids.ravel()
    T, k = topk_ids.shape
    pad = T * k
    cnt = np.bincount(flat, minlength=E)
    padded = (cnt + bs - 1) // bs * bs
    off = np.concatenate([[0], np.cumsum(padded)])
    max_padded = T * k + E * (bs - 1)
    sorted_ids = np.full(max_padded, pad, np.int32)
    order = np.argsort(flat, kind="stable")
    rank = np.arange(order.size) - np.repeat(np.cumsum(cnt) - cnt, cnt)
    sorted_ids[off[flat[order]] + rank] = order
    experts = np.zeros(max_padded // bs, np.int32)
    experts[: off[-1] // bs] = np.repeat(np.arange(E), padded // bs)
    return sorted_ids, experts, np.int32(off[-1])


def main():
    g = np.random.Generator(np.random.PCG64(20240828))
    out = {}
    # dequant fixtures (a few blocks of each type; nb odd for Q8_0/Q4_0)
    for name, qt, nb, fn in (("q8_0", 8, 7, q8_0_dequant), ("q4_0", 2, 9, q4_0_dequant),
                             ("q4_k", 12, 5, q4_k_dequant)):
        bk = 256 if qt == 12 else 32
        if qt == 8:
            soa = np.concatenate([f16_bits(g.uniform(-0.05, 0.05, nb)).view(np.uint8),
                                  g.integers(-128, 128, nb * 32, dtype=np.int8).view(np.uint8)])
        elif qt == 2:
            soa = np.concatenate([f16_bits(g.uniform(-0.05, 0.05, nb)).view(np.uint8),
                                  g.integers(0, 256, nb * 16, dtype=np.uint8)])
        else:
            hdr = g.integers(0, 256, (nb, 16), dtype=np.uint8)
            hdr[:, 0:4] = np.stack([f16_bits(g.uniform(0.001, 0.05, nb)),
                                    f16_bits(g.uniform(0.0, 0.05, nb))], 1).view(np.uint8).reshape(nb, 4)
            soa = np.concatenate([hdr.ravel(), g.integers(0, 256, nb * 128, dtype=np.uint8)])
        f32, f16, bf = fn(soa, nb)
        out[f"{name}_soa"] = soa
        out[f"{name}_f32"] = f32
        out[f"{name}_f16"] = f16
        out[f"{name}_bf16"] = bf
        assert f32.size == nb * bk
    # activation quantizers (include exact ties and zero blocks)
    x = g.standard_normal(512).astype(np.float32)
    x[32:64] = 0.0
    x[64:96] = np.linspace(-127, 127, 32).astype(np.float32)
    x[256:512] *= 3.0
    d0, q0 = quant_q8_0(x)
    out["act_x"] = x
    out["q8_0_d"], out["q8_0_q"] = d0, q0.ravel()
    dk, qk, bk = quant_q8_k(x)
    out["q8_k_d"], out["q8_k_q"], out["q8_k_bs"] = dk, qk.ravel(), bk.ravel()
    # qmatmul (Candle method) on small shapes
    for name, qt, N, K in (("mm_q4_0", 2, 24, 256), ("mm_q8_0", 8, 24, 256),
                           ("mm_q4_k", 12, 24, 512)):
        bk_ = 256 if qt == 12 else 32
        nb = N * K // bk_
        if qt == 12:
            hdr = g.integers(0, 256, (nb, 16), dtype=np.uint8)
            hdr[:, 0:4] = np.stack([f16_bits(g.uniform(0.001, 0.02, nb)),
                                    f16_bits(g.uniform(0.001, 0.02, nb))], 1).view(np.uint8).reshape(nb, 4)
            soa = np.concatenate([hdr.ravel(), g.integers(0, 256, nb * 128, dtype=np.uint8)])
        elif qt == 8:
            soa = np.concatenate([f16_bits(g.uniform(0.001, 0.02, nb)).view(np.uint8),
                                  g.integers(-127, 128, nb * 32, dtype=np.int8).view(np.uint8)])
        else:
            soa = np.concatenate([f16_bits(g.uniform(0.001, 0.02, nb)).view(np.uint8),
                                  g.integers(0, 256, nb * 16, dtype=np.uint8)])
        xa = g.standard_normal((3, K)).astype(np.float32)
        out[f"{name}_w"], out[f"{name}_x"] = soa, xa
        out[f"{name}_y"] = qmatmul(qt, soa, xa, N, K)
        out[f"{name}_shape"] = np.array([N, K], np.int32)
    # MoE routing
    logits = g.standard_normal((16, 32)).astype(np.float32)
    w, idx = topk_softmax(logits, 4, True)
    out["topk_logits"], out["topk_w"], out["topk_idx"] = logits, w, idx
    w2, idx2 = topk_softmax(logits, 4, False)
    out["topk_w_nonorm"], out["topk_idx_nonorm"] = w2, idx2
    ids = g.integers(0, 8, (13, 3)).astype(np.int32)
    s, e, n = moe_align(ids, 8, 4)
    out["align_ids"], out["align_sorted"], out["align_experts"] = ids, s, e
    out["align_ntpp"] = np.array([n], np.int32)
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **out)
    print("wrote", os.path.join(HERE, "golden.npz"), len(out), "arrays")


if __name__ == "__main__":
    main()
