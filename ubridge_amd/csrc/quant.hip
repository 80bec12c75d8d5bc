// quant.hip -- GGUF block dequant / quantize kernels for gfx950.
//
// Device layout is the reference's "SoA" form (quant.cpp:217-220,439-442):
// one contiguous array of block headers (scales) followed by one contiguous
// array of block payloads.  For an [N, K] weight, blocks run row-major along K.
//   Q8_0: [nb x fp16 d][nb x 32 int8]
//   Q4_0: [nb x fp16 d][nb x 16 B]            (GGML nibble order)
//   Q4_K: [nb x 16 B {fp16 d, fp16 dmin, u8 sc[12]}][nb x 128 B]
// All kernels are plain HBM streams: 16-byte vector loads, one pass.
#include "common.h"

namespace {

constexpr int kThreads = 256;

inline int grid_for(size_t work, int per_block = kThreads) {
  size_t g = (work + per_block - 1) / per_block;
  if (g > 65535u * 16u) g = 65535u * 16u;  // grid-stride beyond this
  return (int)(g == 0 ? 1 : g);
}

// ------------------------------------------------- Q8_0 / Q4_0 dequant
// 16 output bytes per item (E = 8 elements of a 16-bit T, 4 of f32), item i
// = elements [E i, E i + E), so a wave's store is one contiguous run; a lane
// takes kFlatU items 256 apart, loads first.  Block b = E i / 32, t = i mod
// (32 / E):
//   Q8_0: codes bytes [E t, E t + E) of the block's 32.  f32/f16: T(d*q), one
//     rounding of the exact product.  bf16: the reference converts the fp16
//     scale to bf16 before the multiply (quant.cpp:250): bf16(bf16(d) * q).
//   Q4_0: element e < 16 is the low nibble of byte e, e >= 16 the high nibble
//     of byte e - 16; y = (c - 8) * d.
constexpr int kFlatU = 4;
template <int QT, int DT>
__global__ void __launch_bounds__(kThreads) k_dequant_flat(const uint8_t* __restrict__ in, const uint8_t* __restrict__ body,
                                                           void* __restrict__ out, size_t nb) {
  constexpr int E = DT == UB_F32 ? 4 : 8, IPB = 32 / E, PB = QT == UB_Q8_0 ? 32 : 16;
  const uint16_t* dptr = (const uint16_t*)in;
  const size_t ni = nb * IPB;
  for (size_t i0 = blockIdx.x * (size_t)(kThreads * kFlatU) + threadIdx.x; i0 < ni;
       i0 += (size_t)gridDim.x * (kThreads * kFlatU)) {
    uint16_t dh[kFlatU];
    uint32_t c[kFlatU][2];
#pragma unroll
    for (int u = 0; u < kFlatU; u++) {
      const size_t i = i0 + (size_t)u * kThreads;
      if (i >= ni) break;
      const size_t b = i / IPB;
      const int t = (int)(i % IPB);
      dh[u] = dptr[b];
      const int off = QT == UB_Q8_0 ? E * t : E * t % 16;
      const uint8_t* q = body + b * PB + off;
      if constexpr (E == 8) {
        const uint2 v = *(const uint2*)q;
        c[u][0] = v.x, c[u][1] = v.y;
      } else {
        c[u][0] = *(const uint32_t*)q, c[u][1] = 0;
      }
    }
#pragma unroll
    for (int u = 0; u < kFlatU; u++) {
      const size_t i = i0 + (size_t)u * kThreads;
      if (i >= ni) break;
      float d = ub_f16_to_f32(dh[u]);
      float y[E];
      if constexpr (QT == UB_Q8_0) {
        if constexpr (DT == UB_BF16) d = ub_bf16_to_f32(ub_f32_to_bf16(d));
#pragma unroll
        for (int l = 0; l < E; l++) y[l] = d * (float)(int8_t)(c[u][l >> 2] >> (8 * (l & 3)));
      } else {
        const int sh = E * (int)(i % IPB) >= 16 ? 4 : 0;
#pragma unroll
        for (int l = 0; l < E; l++)
          y[l] = (float)((int)((c[u][l >> 2] >> (8 * (l & 3) + sh)) & 15) - 8) * d;
      }
      if constexpr (DT == UB_F32) {
        ((float4*)out)[i] = make_float4(y[0], y[1], y[2], y[3]);
      } else {
        uint32_t p[4];
#pragma unroll
        for (int l = 0; l < 4; l++) {
          const uint16_t lo = DT == UB_F16 ? ub_f32_to_f16(y[2 * l]) : ub_f32_to_bf16(y[2 * l]);
          const uint16_t hi =
              DT == UB_F16 ? ub_f32_to_f16(y[2 * l + 1]) : ub_f32_to_bf16(y[2 * l + 1]);
          p[l] = lo | ((uint32_t)hi << 16);
        }
        ((uint4*)out)[i] = make_uint4(p[0], p[1], p[2], p[3]);
      }
    }
  }
}

// ------------------------------------------- unaligned-payload fallback
// One lane per element; used only when the payload array of a Q8_0/Q4_0
// tensor does not start on a 16-byte boundary (an odd block count).
template <int QT, int DT>
__global__ void __launch_bounds__(kThreads) k_dequant_scalar(const uint8_t* __restrict__ in, const uint8_t* __restrict__ body,
                                                             void* __restrict__ out, size_t nb) {
  const uint16_t* dptr = (const uint16_t*)in;
  const uint8_t* q = body;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < nb * 32;
       i += (size_t)gridDim.x * blockDim.x) {
    size_t b = i >> 5;
    int e = (int)(i & 31);
    float d = ub_f16_to_f32(dptr[b]);
    float v;
    if constexpr (QT == UB_Q8_0) {
      if constexpr (DT == UB_BF16) d = ub_bf16_to_f32(ub_f32_to_bf16(d));
      v = d * (float)(int8_t)q[i];
    } else {
      uint8_t c = q[b * 16 + (e & 15)];
      v = (float)((int)(e < 16 ? (c & 15) : (c >> 4)) - 8) * d;
    }
    ub_store<DT>(out, i, v);
  }
}

// ------------------------------------------------------------ Q4_K dequant
// 16 output bytes per lane and step (E = 8 elements of a 16-bit T, 4 of
// f32), so a wave's store is one contiguous run: item i of a 256-element
// block b = i / (256 / E) owns elements [E t, E t + E), t = i mod (256 / E),
// of sub-block s = E t / 32, whose codes are the low (s even) or high (s odd)
// nibbles of bytes 32 (s / 2) + (E t mod 32) on.  A lane takes kQ4kU items
// 256 apart, loads first, so that enough bytes are in flight per lane.
// y = d*sc*q - dmin*m; d*sc*q is exact in f32 so fma or not is the same.
constexpr int kQ4kU = 4;
template <int DT>
__global__ void __launch_bounds__(kThreads) k_dequant_q4_k(const uint8_t* __restrict__ in, const uint8_t* __restrict__ body,
                                                           void* __restrict__ out, size_t nb) {
  constexpr int E = DT == UB_F32 ? 4 : 8, LPB = 256 / E;
  const uint4* hdr = (const uint4*)in;
  const size_t nl = nb * LPB;
  for (size_t i0 = blockIdx.x * (size_t)(kThreads * kQ4kU) + threadIdx.x; i0 < nl;
       i0 += (size_t)gridDim.x * (kThreads * kQ4kU)) {
    uint4 hd[kQ4kU];
    uint32_t c[kQ4kU][E / 4];
#pragma unroll
    for (int u = 0; u < kQ4kU; u++) {
      const size_t i = i0 + (size_t)u * kThreads;
      if (i >= nl) break;
      const size_t b = i / LPB;
      const int t = (int)(i % LPB), sb = E * t / 32;
      hd[u] = hdr[b];
      const uint8_t* q = body + b * 128 + 32 * (sb >> 1) + E * t % 32;
      if constexpr (E == 8) {
        const uint2 v = *(const uint2*)q;
        c[u][0] = v.x, c[u][1] = v.y;
      } else {
        c[u][0] = *(const uint32_t*)q;
      }
    }
#pragma unroll
    for (int u = 0; u < kQ4kU; u++) {
      const size_t i = i0 + (size_t)u * kThreads;
      if (i >= nl) break;
      const int sb = E * (int)(i % LPB) / 32;
      int sc, m;
      q4k_scale_min(sb, hd[u].y, hd[u].z, hd[u].w, sc, m);
      const float d1 = ub_f16_to_f32((uint16_t)(hd[u].x & 0xffff)) * (float)sc;
      const float m1 = ub_f16_to_f32((uint16_t)(hd[u].x >> 16)) * (float)m;
      const int sh = 4 * (sb & 1);
      float y[E];
#pragma unroll
      for (int l = 0; l < E; l++)
        y[l] = d1 * (float)((c[u][l >> 2] >> (8 * (l & 3) + sh)) & 15) - m1;
      if constexpr (DT == UB_F32) {
        ((float4*)out)[i] = make_float4(y[0], y[1], y[2], y[3]);
      } else {
        uint32_t p[4];
#pragma unroll
        for (int l = 0; l < 4; l++) {
          const uint16_t lo = DT == UB_F16 ? ub_f32_to_f16(y[2 * l]) : ub_f32_to_bf16(y[2 * l]);
          const uint16_t hi =
              DT == UB_F16 ? ub_f32_to_f16(y[2 * l + 1]) : ub_f32_to_bf16(y[2 * l + 1]);
          p[l] = lo | ((uint32_t)hi << 16);
        }
        ((uint4*)out)[i] = make_uint4(p[0], p[1], p[2], p[3]);
      }
    }
  }
}

// ------------------------------------------------- Q8_0 quantize (32-blocks)
// Candle / GGML from_float: amax over the whole block, d = amax/127,
// q = round-half-away(x * (1/d)).  One lane per block.  MODE 0 writes the
// reference SoA layout [nb x fp16 d][nb x 32 int8]; MODE 1 writes the GEMV
// workspace (int8 codes, f32 copy of the fp16-rounded d, and the int32 sum of
// the block's first 16 codes, which the Q4_0 dot needs for its low nibbles).
template <int DT, int MODE>
__global__ void __launch_bounds__(kThreads) k_quantize_q8_0(const void* __restrict__ x,
                                                            uint8_t* __restrict__ out, size_t nb,
                                                            float* __restrict__ dws,
                                                            int* __restrict__ sws) {
  for (size_t b = blockIdx.x * (size_t)blockDim.x + threadIdx.x; b < nb;
       b += (size_t)gridDim.x * blockDim.x) {
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; j++) v[j] = ub_load<DT>(x, b * 32 + j);
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    float d = __fdiv_rn(amax, 127.0f);
    float id = d != 0.f ? __fdiv_rn(1.0f, d) : 0.f;
    uint16_t dh = ub_f32_to_f16(d);
    int8_t q[32];
    int s = 0;
#pragma unroll
    for (int j = 0; j < 32; j++) {
      q[j] = (int8_t)roundf(__fmul_rn(v[j], id));
      if (j < 16) s += q[j];
    }
    if constexpr (MODE == 0) {
      ((uint16_t*)out)[b] = dh;
      uint4* o = (uint4*)(out + nb * 2 + b * 32);
      o[0] = *(uint4*)&q[0];
      o[1] = *(uint4*)&q[16];
    } else {
      uint4* o = (uint4*)(out + b * 32);
      o[0] = *(uint4*)&q[0];
      o[1] = *(uint4*)&q[16];
      dws[b] = ub_f16_to_f32(dh);
      sws[b] = s;
    }
  }
}

// The same quantization, eight lanes per block: each lane loads 4
// consecutive elements (one 8- or 16-byte load), the block's amax is a
// 3-step shuffle, every lane of the group derives the same d and 1/d, writes
// its 4 codes as one dword and lanes 0-3 sum the first 16 codes.  Identical
// values to k_quantize_q8_0 (max is exact, the arithmetic per element is the
// same); 8x the lanes and coalesced accesses.  x must be aligned to its 4
// elements (16 / 8 bytes) and the codes to 4 bytes: MODE 0 writes the SoA
// layout (codes at out + 2 nb), MODE 1 the GEMV workspace.
template <int DT, int MODE>
__global__ void __launch_bounds__(kThreads) k_quantize_q8_0_v(const void* __restrict__ x,
                                                              uint8_t* __restrict__ out, size_t nb,
                                                              float* __restrict__ dws,
                                                              int* __restrict__ sws) {
  int8_t* q = (int8_t*)(MODE == 0 ? out + nb * 2 : out);
  const int l8 = threadIdx.x & 7;
  for (size_t b = (blockIdx.x * (size_t)kThreads + threadIdx.x) >> 3; b < nb;
       b += (size_t)gridDim.x * (kThreads / 8)) {
    float v[4];
    if constexpr (DT == UB_F32) {
      const float4 f = ((const float4*)x)[b * 8 + l8];
      v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
    } else if constexpr (DT == UB_F16) {
      const uint2 u = ((const uint2*)x)[b * 8 + l8];
      v[0] = ub_f16_to_f32((uint16_t)(u.x & 0xffff));
      v[1] = ub_f16_to_f32((uint16_t)(u.x >> 16));
      v[2] = ub_f16_to_f32((uint16_t)(u.y & 0xffff));
      v[3] = ub_f16_to_f32((uint16_t)(u.y >> 16));
    } else {
      const uint2 u = ((const uint2*)x)[b * 8 + l8];
      v[0] = __uint_as_float(u.x << 16);
      v[1] = __uint_as_float(u.x & 0xffff0000u);
      v[2] = __uint_as_float(u.y << 16);
      v[3] = __uint_as_float(u.y & 0xffff0000u);
    }
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = d != 0.f ? __fdiv_rn(1.0f, d) : 0.f;
    uint32_t w = 0;
    int sq = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int c = (int)roundf(__fmul_rn(v[j], id));
      w |= (uint32_t)(c & 0xff) << (8 * j);
      sq += c;
    }
    ((uint32_t*)q)[b * 8 + l8] = w;
    sq = l8 < 4 ? sq : 0;  // the first 16 codes are lanes 0-3's
    sq += __shfl_xor(sq, 1, 64);
    sq += __shfl_xor(sq, 2, 64);
    if (l8 == 0) {
      if constexpr (MODE == 0) {
        ((uint16_t*)out)[b] = ub_f32_to_f16(d);
      } else {
        dws[b] = ub_f16_to_f32(ub_f32_to_f16(d));
        sws[b] = sq;
      }
    }
  }
}

// ------------------------------------------------- Q8_K quantize (256-blocks)
// Candle BlockQ8K::from_float: max = signed value with the largest |x| (first
// index wins a tie), iscale = -128/max, q = min(127, round(iscale*x)),
// d = 1/iscale.  One wavefront per block, 4 consecutive elements per lane;
// the (|x|, index) arg-max is a wave reduction.  Writes the codes, d and the
// 32-element code sums the Q4_K GEMV uses.
template <int DT>
__global__ void __launch_bounds__(256) k_quantize_q8_k(const void* __restrict__ x,
                                                       int8_t* __restrict__ qout, size_t nb,
                                                       float* __restrict__ dout,
                                                       int* __restrict__ sum32) {
  const int lane = threadIdx.x & 63;
  size_t b = blockIdx.x * (size_t)(blockDim.x / 64) + (threadIdx.x >> 6);
  if (b >= nb) return;
  float v[4];
  if constexpr (DT == UB_F32) {
    const float4 f = *(const float4*)((const float*)x + b * 256 + lane * 4);
    v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
  } else {
    const uint2 u = *(const uint2*)((const uint16_t*)x + b * 256 + lane * 4);
    v[0] = __uint_as_float(u.x << 16);
    v[1] = __uint_as_float(u.x & 0xffff0000u);
    v[2] = __uint_as_float(u.y << 16);
    v[3] = __uint_as_float(u.y & 0xffff0000u);
  }
  float amax = 0.f;
  int aidx = 1 << 30;
  float mx = 0.f;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    float a = fabsf(v[j]);
    if (amax < a) { amax = a; aidx = lane * 4 + j; mx = v[j]; }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    float oa = __shfl_xor(amax, off, 64);
    int oi = __shfl_xor(aidx, off, 64);
    float om = __shfl_xor(mx, off, 64);
    if (oa > amax || (oa == amax && oi < aidx)) { amax = oa; aidx = oi; mx = om; }
  }
  int q[4] = {0, 0, 0, 0};
  float d = 0.f;
  if (amax != 0.f) {
    float iscale = __fdiv_rn(-128.0f, mx);
#pragma unroll
    for (int j = 0; j < 4; j++) q[j] = (int)fminf(roundf(__fmul_rn(iscale, v[j])), 127.f);
    d = __fdiv_rn(1.0f, iscale);
  }
  *(uint32_t*)(qout + b * 256 + lane * 4) = (q[0] & 0xff) | ((q[1] & 0xff) << 8) |
                                            ((q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
  int s = q[0] + q[1] + q[2] + q[3];
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  s += __shfl_xor(s, 4, 64);
  if ((lane & 7) == 0) sum32[b * 8 + (lane >> 3)] = s;
  if (lane == 0) dout[b] = d;
}

// ------------------------------------------------------ AoS <-> SoA repack
template <int HEAD, int BODY, bool TO_SOA>
__global__ void __launch_bounds__(kThreads) k_repack(const uint8_t* __restrict__ src,
                                                     uint8_t* __restrict__ dst, size_t nb) {
  // one output byte per thread and pass: a wavefront writes 64 consecutive
  // bytes and reads 64 mostly consecutive ones (the block sizes, 18 / 34 /
  // 144 bytes, leave AoS blocks unaligned for wider accesses)
  constexpr size_t BS = HEAD + BODY;
  const size_t total = nb * BS;
  for (size_t o = blockIdx.x * (size_t)blockDim.x + threadIdx.x; o < total;
       o += (size_t)gridDim.x * blockDim.x) {
    size_t from;
    if constexpr (TO_SOA) {  // o in [headers | payloads]
      if (o < nb * HEAD) from = o / HEAD * BS + o % HEAD;
      else from = (o - nb * HEAD) / BODY * BS + HEAD + (o - nb * HEAD) % BODY;
    } else {  // o in the AoS blocks
      const size_t b = o / BS, j = o % BS;
      from = j < HEAD ? b * HEAD + j : nb * HEAD + b * BODY + (j - HEAD);
    }
    dst[o] = src[from];
  }
}

// Blocks [b0, b0 + nb) of a SoA tensor of nb_total blocks (headers, then
// payloads), dequantized to out[0 .. nb * block).
template <int QT>
int dequant_part(const uint8_t* w, size_t nb_total, size_t b0, size_t nb, void* out, int dt,
                 hipStream_t s, const char* nm) {
  constexpr int HB = QT == UB_Q4_K ? 16 : 2, PB = QT == UB_Q4_K ? 128 : QT == UB_Q8_0 ? 32 : 16;
  if (nb == 0) return UB_OK;
  const uint8_t* hd = w + b0 * HB;
  const uint8_t* body = w + nb_total * HB + b0 * PB;
  if constexpr (QT != UB_Q4_K) {
    if (((uintptr_t)body & 15) != 0 || ((uintptr_t)hd & 1) != 0) {
      int g = grid_for(nb * 32);
      if (dt == UB_F32) k_dequant_scalar<QT, UB_F32><<<g, kThreads, 0, s>>>(hd, body, out, nb);
      else if (dt == UB_F16) k_dequant_scalar<QT, UB_F16><<<g, kThreads, 0, s>>>(hd, body, out, nb);
      else k_dequant_scalar<QT, UB_BF16><<<g, kThreads, 0, s>>>(hd, body, out, nb);
      return ub_check_launch(nm);
    }
  }
  if constexpr (QT != UB_Q4_K) {
    int g = grid_for(nb * (dt == UB_F32 ? 8 : 4), kThreads * kFlatU);
    if (dt == UB_F32) k_dequant_flat<QT, UB_F32><<<g, kThreads, 0, s>>>(hd, body, out, nb);
    else if (dt == UB_F16) k_dequant_flat<QT, UB_F16><<<g, kThreads, 0, s>>>(hd, body, out, nb);
    else k_dequant_flat<QT, UB_BF16><<<g, kThreads, 0, s>>>(hd, body, out, nb);
  } else {
    int g = grid_for(nb * (dt == UB_F32 ? 64 : 32), kThreads * kQ4kU);
    if (dt == UB_F32) k_dequant_q4_k<UB_F32><<<g, kThreads, 0, s>>>(hd, body, out, nb);
    else if (dt == UB_F16) k_dequant_q4_k<UB_F16><<<g, kThreads, 0, s>>>(hd, body, out, nb);
    else k_dequant_q4_k<UB_BF16><<<g, kThreads, 0, s>>>(hd, body, out, nb);
  }
  return ub_check_launch(nm);
}

template <int QT>
int dequant_launch(const void* in, void* out, size_t numel, int dt, void* stream, const char* nm) {
  constexpr int bk = QT == UB_Q4_K ? 256 : 32;
  UB_REQUIRE(numel % bk == 0, "%s: numel %zu is not a multiple of %d", nm, numel, bk);
  if (numel == 0) return UB_OK;
  UB_REQUIRE(in && out, "%s: null pointer", nm);
  const size_t nb = numel / bk;
  if constexpr (QT != UB_Q4_K)  // the scalar kernel also for a misaligned header array
    if (((uintptr_t)in & 15) != 0) {
      const uint8_t* i8 = (const uint8_t*)in;
      int g = grid_for(nb * 32);
      hipStream_t s = ub_stream(stream);
      if (dt == UB_F32) k_dequant_scalar<QT, UB_F32><<<g, kThreads, 0, s>>>(i8, i8 + nb * 2, out, nb);
      else if (dt == UB_F16) k_dequant_scalar<QT, UB_F16><<<g, kThreads, 0, s>>>(i8, i8 + nb * 2, out, nb);
      else k_dequant_scalar<QT, UB_BF16><<<g, kThreads, 0, s>>>(i8, i8 + nb * 2, out, nb);
      return ub_check_launch(nm);
    }
  return dequant_part<QT>((const uint8_t*)in, nb, 0, nb, out, dt, ub_stream(stream), nm);
}

template <int DT>
int quantize_q8_0_launch(const void* in, int8_t* out, size_t in_bytes, size_t out_bytes,
                         void* stream, const char* nm) {
  constexpr size_t es = DT == UB_F32 ? 4 : 2;
  size_t n = in_bytes / es;
  if (n == 0) return UB_OK;
  UB_REQUIRE(in && out, "%s: null pointer", nm);
  UB_REQUIRE(n % 32 == 0, "%s: %zu elements is not a multiple of 32", nm, n);
  size_t nb = n / 32;
  UB_REQUIRE(out_bytes >= nb * 34, "%s: output holds %zu bytes, needs %zu", nm, out_bytes, nb * 34);
  if (nb == 0) return UB_OK;
  // eight lanes per block when the loads and code stores are aligned
  if (((uintptr_t)in & (4 * es - 1)) == 0 && (((uintptr_t)out + nb * 2) & 3) == 0)
    k_quantize_q8_0_v<DT, 0><<<grid_for(nb * 8), kThreads, 0, ub_stream(stream)>>>(
        in, (uint8_t*)out, nb, nullptr, nullptr);
  else
    k_quantize_q8_0<DT, 0><<<grid_for(nb), kThreads, 0, ub_stream(stream)>>>(
        in, (uint8_t*)out, nb, nullptr, nullptr);
  return ub_check_launch(nm);
}

}  // namespace

// Rows [r0, r0 + nrows) of a SoA GGUF weight [N, K] (qtype 2 / 8 / 12)
// dequantized to out [nrows, K] in dtype dt: the values of dequantize_block_*.
int ub_dequant_rows(int qtype, const void* w, int N, int K, int r0, int nrows, void* out, int dt,
                    hipStream_t s) {
  const int bk = qtype == UB_Q4_K ? 256 : 32;
  const size_t nbr = (size_t)K / bk, nbt = (size_t)N * nbr;
  const uint8_t* w8 = (const uint8_t*)w;
  const char* nm = "dequantize rows";
  if (qtype == UB_Q4_K) return dequant_part<UB_Q4_K>(w8, nbt, r0 * nbr, nrows * nbr, out, dt, s, nm);
  if (qtype == UB_Q8_0) return dequant_part<UB_Q8_0>(w8, nbt, r0 * nbr, nrows * nbr, out, dt, s, nm);
  return dequant_part<UB_Q4_0>(w8, nbt, r0 * nbr, nrows * nbr, out, dt, s, nm);
}

// ====================================================================== ABI
// dequantize_block_q8_0_{f16,bf16,f32}(int8_t* in, T* out, size_t numel)
// replaces quant.cpp:257-268 (names: device_executor.rs:299-301).
#define UB_DEQ(NAME, QT, DT)                                                  \
  UB_API void NAME(const int8_t* in, void* out, size_t numel, void* stream) { \
    dequant_launch<QT>(in, out, numel, DT, stream, #NAME);                     \
  }
UB_DEQ(dequantize_block_q8_0_f16, UB_Q8_0, UB_F16)
UB_DEQ(dequantize_block_q8_0_bf16, UB_Q8_0, UB_BF16)
UB_DEQ(dequantize_block_q8_0_f32, UB_Q8_0, UB_F32)
UB_DEQ(dequantize_block_q4_k_f16, UB_Q4_K, UB_F16)
UB_DEQ(dequantize_block_q4_k_bf16, UB_Q4_K, UB_BF16)
UB_DEQ(dequantize_block_q4_k_f32, UB_Q4_K, UB_F32)
UB_DEQ(dequantize_block_q4_0_f16, UB_Q4_0, UB_F16)
UB_DEQ(dequantize_block_q4_0_bf16, UB_Q4_0, UB_BF16)
UB_DEQ(dequantize_block_q4_0_f32, UB_Q4_0, UB_F32)
#undef UB_DEQ

// quantize_block_q8_0_{bf16,f16,f32}(T* in, int8_t* out, size_t in_bytes,
// size_t out_bytes) replaces quant.cpp:341-353.
UB_API void quantize_block_q8_0_bf16(const void* in, int8_t* out, size_t ib, size_t ob, void* s) {
  quantize_q8_0_launch<UB_BF16>(in, out, ib, ob, s, "quantize_block_q8_0_bf16");
}
UB_API void quantize_block_q8_0_f16(const void* in, int8_t* out, size_t ib, size_t ob, void* s) {
  quantize_q8_0_launch<UB_F16>(in, out, ib, ob, s, "quantize_block_q8_0_f16");
}
UB_API void quantize_block_q8_0_f32(const void* in, int8_t* out, size_t ib, size_t ob, void* s) {
  quantize_q8_0_launch<UB_F32>(in, out, ib, ob, s, "quantize_block_q8_0_f32");
}
// quantize_block_q4_k_* (quant.cpp:644-657): the reference kernel's quantize
// call is commented out (quant.cpp:639), so it writes no codes.  Kept as a
// named entry that reports UB_ERR_UNSUPPORTED rather than writing garbage.
#define UB_QK(NAME)                                                                   \
  UB_API void NAME(const void*, int8_t*, size_t, size_t, void*) {                     \
    ub_set_error(UB_ERR_UNSUPPORTED, #NAME ": Q4_K quantization is not implemented"); \
  }
UB_QK(quantize_block_q4_k_bf16)
UB_QK(quantize_block_q4_k_f16)
UB_QK(quantize_block_q4_k_f32)
#undef UB_QK

// GGUF AoS <-> reference SoA repack (no reference counterpart: the loader
// side of the format, so GGUF files can feed the SoA kernels).
UB_API int ubridge_gguf_to_soa(int qtype, const void* aos, void* soa, size_t nblocks, void* stream) {
  UB_REQUIRE(aos && soa && aos != soa, "ubridge_gguf_to_soa: bad pointers");
  if (nblocks == 0) return UB_OK;
  hipStream_t s = ub_stream(stream);
  const int g = grid_for(nblocks * (qtype == UB_Q4_K ? 144 : qtype == UB_Q8_0 ? 34 : 18));
  const uint8_t* a = (const uint8_t*)aos;
  uint8_t* o = (uint8_t*)soa;
  if (qtype == UB_Q4_0) k_repack<2, 16, true><<<g, kThreads, 0, s>>>(a, o, nblocks);
  else if (qtype == UB_Q8_0) k_repack<2, 32, true><<<g, kThreads, 0, s>>>(a, o, nblocks);
  else if (qtype == UB_Q4_K) k_repack<16, 128, true><<<g, kThreads, 0, s>>>(a, o, nblocks);
  else return ub_set_error(UB_ERR_UNSUPPORTED, "ubridge_gguf_to_soa: qtype %d", qtype);
  return ub_check_launch("ubridge_gguf_to_soa");
}
UB_API int ubridge_soa_to_gguf(int qtype, const void* soa, void* aos, size_t nblocks, void* stream) {
  UB_REQUIRE(aos && soa && aos != soa, "ubridge_soa_to_gguf: bad pointers");
  if (nblocks == 0) return UB_OK;
  hipStream_t s = ub_stream(stream);
  const int g = grid_for(nblocks * (qtype == UB_Q4_K ? 144 : qtype == UB_Q8_0 ? 34 : 18));
  const uint8_t* a = (const uint8_t*)soa;
  uint8_t* o = (uint8_t*)aos;
  if (qtype == UB_Q4_0) k_repack<2, 16, false><<<g, kThreads, 0, s>>>(a, o, nblocks);
  else if (qtype == UB_Q8_0) k_repack<2, 32, false><<<g, kThreads, 0, s>>>(a, o, nblocks);
  else if (qtype == UB_Q4_K) k_repack<16, 128, false><<<g, kThreads, 0, s>>>(a, o, nblocks);
  else return ub_set_error(UB_ERR_UNSUPPORTED, "ubridge_soa_to_gguf: qtype %d", qtype);
  return ub_check_launch("ubridge_soa_to_gguf");
}

// ------------------------------------------------ internal: GEMV activations
// Used by gemv.hip.  x: [M, K] f32 or bf16.
int ub_quantize_act_q8_0(const void* x, int x_dt, size_t n, int8_t* q, float* d, int* s,
                         hipStream_t st) {
  size_t nb = n / 32;
  if (((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 3) == 0) {  // eight lanes per block
    const int g = grid_for(nb * 8);
    if (x_dt == UB_F32) k_quantize_q8_0_v<UB_F32, 1><<<g, kThreads, 0, st>>>(x, (uint8_t*)q, nb, d, s);
    else k_quantize_q8_0_v<UB_BF16, 1><<<g, kThreads, 0, st>>>(x, (uint8_t*)q, nb, d, s);
  } else if (x_dt == UB_F32) {
    k_quantize_q8_0<UB_F32, 1><<<grid_for(nb), kThreads, 0, st>>>(x, (uint8_t*)q, nb, d, s);
  } else {
    k_quantize_q8_0<UB_BF16, 1><<<grid_for(nb), kThreads, 0, st>>>(x, (uint8_t*)q, nb, d, s);
  }
  return ub_check_launch("quantize activations q8_0");
}
int ub_quantize_act_q8_k(const void* x, int x_dt, size_t n, int8_t* q, float* d, int* bs,
                         hipStream_t st) {
  size_t nb = n / 256;
  int g = (int)((nb + 3) / 4);
  if (x_dt == UB_F32) k_quantize_q8_k<UB_F32><<<g, kThreads, 0, st>>>(x, q, nb, d, bs);
  else k_quantize_q8_k<UB_BF16><<<g, kThreads, 0, st>>>(x, q, nb, d, bs);
  return ub_check_launch("quantize activations q8_k");
}

// ------------------------------------------------- name-keyed launch thunks
#include "registry.h"
#define UB_DEQ_THUNK(NAME)                                                    \
  void ub_thunk_##NAME(void** args, void* stream) {                          \
    NAME(UB_ARG(const int8_t*, 0), UB_ARG(void*, 1), UB_ARG(size_t, 2), stream); \
  }
#define UB_Q_THUNK(NAME)                                                          \
  void ub_thunk_##NAME(void** args, void* stream) {                              \
    NAME(UB_ARG(const void*, 0), UB_ARG(int8_t*, 1), UB_ARG(size_t, 2), UB_ARG(size_t, 3), \
         stream);                                                                 \
  }
UB_DEQ_THUNK(dequantize_block_q8_0_f16)
UB_DEQ_THUNK(dequantize_block_q8_0_bf16)
UB_DEQ_THUNK(dequantize_block_q8_0_f32)
UB_DEQ_THUNK(dequantize_block_q4_k_f16)
UB_DEQ_THUNK(dequantize_block_q4_k_bf16)
UB_DEQ_THUNK(dequantize_block_q4_k_f32)
UB_DEQ_THUNK(dequantize_block_q4_0_f16)
UB_DEQ_THUNK(dequantize_block_q4_0_bf16)
UB_DEQ_THUNK(dequantize_block_q4_0_f32)
UB_Q_THUNK(quantize_block_q8_0_f16)
UB_Q_THUNK(quantize_block_q8_0_bf16)
UB_Q_THUNK(quantize_block_q8_0_f32)
UB_Q_THUNK(quantize_block_q4_k_f16)
UB_Q_THUNK(quantize_block_q4_k_bf16)
UB_Q_THUNK(quantize_block_q4_k_f32)
