// gemm.hip -- weight-only quantized GEMM on CDNA4 MFMA (gfx950).
//
//   C[b, M, N] = A[b, M, K] . deq(W)[K, N],  A / C bf16 or f16, f32 accumulate
//
// One MFMA core, several weight producers.  Per K-step of 64 every thread
// turns one 4-column x 8-k slab of the packed weight into T (bf16 / f16) and
// writes it to LDS as N-major rows ([n][k], k contiguous), which is exactly
// the register image one lane feeds to v_mfma_f32_32x32x16_{bf16,f16} for
// B (8 consecutive k of one column) -- so the dequantized weight tile never
// exists in HBM.  Producers:
//   W_GPTQ4   int32 [K/8, N] (8 K-consecutive nibbles, LSB first), scales
//             T [K/g, N], zeros int32 [K/g, N/8] (8 N-consecutive nibbles):
//             w = T((q - z) * s)                         (north-star W4A16)
//   W_U4REF   uint8 [K/2, N] (low nibble = even k), scales and zeros T [K/g, N]:
//             w = T(((float)q - z) * s)   (matmul_{bf16,f16}_4bit layout,
//             kernels/matmul.cpp:613-620,678-679)
//   W_I8_KN / W_I8_NK  int8 [K, N] / [N, K], scales T [K/g, N]:
//             w = T(q * s)                (matmul_*_8bit, matmul_decoding.h:451-471)
//   W_DENSE_KN / W_DENSE_NK  T [K, N] / [N, K]   (matmul_{bf16,f16})
//
// Tiling: 128 x 128 or 256 x 256 block tile, 4 wavefronts in 2 x 2, each a
// grid of MFMA 32x32x16 blocks; BK = 64 with double-buffered LDS; the next
// K-step's global loads are issued before the current step's MFMAs, and all
// global loads are raw buffer loads whose out-of-range lanes read zero (no
// branches, so no forced vmcnt(0) between load issue and MFMA work).  LDS
// fragment reads of the next 16-k substep are interleaved with the current
// substep's MFMAs (sched_group_barrier).
#include "common.h"
#include "registry.h"

#include <stdio.h>
#include <string.h>

#include <map>
#include <memory>
#include <mutex>
#include <string>

// w4a16.hip
int ub_wq_pipelined(int wf, const void* a, const void* w, const void* scales, const void* zeros,
                    void* out, int M, int K, int N, int group, int dtype, int tile, hipStream_t s);
int ub_wq_split(int M, int N, int K);
// blaslt.cpp
bool ub_blaslt_ready(int batch, int M, int N, int K, int rhs_t, int bcast, int ldc, int c_f32,
                     int dt, hipStream_t s);
int ub_blaslt_gemm(const void* a, const void* b, void* c, int batch, int M, int N, int K,
                   int rhs_t, int bcast, int ldc, int c_f32, int dt, hipStream_t s);
// wq_gemv.hip
int ub_copy_b16(const void* x, void* y, size_t n, hipStream_t s);  // gemv.hip
int ub_wq_gemv(int wf, const void* a, const void* w, const void* scales, const void* zeros,
               void* out, int M, int K, int N, int group, int dtype, hipStream_t s);

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

enum { W_GPTQ4 = 0, W_U4REF = 1, W_I8_KN = 2, W_I8_NK = 3, W_DENSE_KN = 4, W_DENSE_NK = 5,
       W_Q40 = 6, W_Q80 = 7, W_Q4K = 8 };
constexpr bool is_gguf(int wf) { return wf == W_Q40 || wf == W_Q80 || wf == W_Q4K; }

constexpr int BK = 64;
constexpr int LDK = BK + 8;  // padded LDS row (elements): conflict-free 16-byte reads
constexpr uint32_t kOOB = 0x80000000u;
constexpr int kRsrcWord3 = 0x00020000;

struct GemmArgs {
  const void* a;
  const void* w;
  const void* scales;
  const void* zeros;
  void* c;
  int M, N, K, group;
  long long sa, sw, sc;  // batch strides (elements of A / bytes of W / elements of C)
  int c_f32;             // C is f32 (else T)
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint64_t bytes) {
  const uint32_t n = bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)n, kRsrcWord3);
}
__device__ __forceinline__ uint4 ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}

template <int DT>
__device__ __forceinline__ float tof(uint32_t bits16) {
  if constexpr (DT == UB_BF16) return __uint_as_float(bits16 << 16);
  else return (float)__builtin_bit_cast(_Float16, (unsigned short)bits16);
}
// two f32 -> packed pair of T (hardware round-to-nearest-even)
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (DT == UB_BF16)
    return (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)lo) |
           ((uint32_t)__builtin_bit_cast(unsigned short, (__bf16)hi) << 16);
  else
    return (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)lo) |
           ((uint32_t)__builtin_bit_cast(unsigned short, (_Float16)hi) << 16);
}

// Raw global data of one thread's weight slab (4 columns x 8 k), loaded one
// K-step ahead and turned into T after the MFMAs of the current step.
struct Slab {
  uint4 q[2];     // packed codes / values (format-specific)
  uint2 s, z;     // 4 scales (T) / 4 zeros (T) or one zeros int32 in z.x
  uint4 d[2];     // dense formats: extra words
  uint4 h[4];     // GGUF formats: the 4 rows' block headers (Q4_K) / scale dwords
};

// Slab (k8, c): 8 k rows starting at k0 + 8*k8, 4 columns starting at n0 + 4*c.
template <int WF, int DT>
__device__ __forceinline__ void load_slab(Slab& S, const GemmArgs& a, __amdgpu_buffer_rsrc_t rw,
                                          __amdgpu_buffer_rsrc_t rs, __amdgpu_buffer_rsrc_t rz,
                                          int k0, int n0, int k8, int c) {
  const int n = n0 + 4 * c, k = k0 + 8 * k8;
  const bool ok = n < a.N && k < a.K;  // N % 4 == 0 and K % 8 == 0 are required by the host
  const int g = (k < a.K ? k : 0) / a.group;
  const uint32_t so = ok ? (uint32_t)((size_t)g * a.N + n) * 2 : kOOB;
  if constexpr (WF == W_GPTQ4) {
    S.q[0] = ld16(rw, ok ? (uint32_t)(((size_t)(k >> 3) * a.N + n) * 4) : kOOB);
    S.s = ld8(rs, so);
    S.z.x = ld4(rz, ok ? (uint32_t)(((size_t)g * (a.N >> 3) + (n >> 3)) * 4) : kOOB);
  } else if constexpr (WF == W_U4REF) {
    // rows k/2 .. k/2+3 of uint8 [K/2, N], 4 bytes each
    const uint32_t base = (uint32_t)((size_t)(k >> 1) * a.N + n);
    S.q[0].x = ld4(rw, ok ? base : kOOB);
    S.q[0].y = ld4(rw, ok ? base + a.N : kOOB);
    S.q[0].z = ld4(rw, ok ? base + 2 * a.N : kOOB);
    S.q[0].w = ld4(rw, ok ? base + 3 * a.N : kOOB);
    S.s = ld8(rs, so);
    S.z = ld8(rz, so);
  } else if constexpr (WF == W_I8_KN) {
    const uint32_t base = (uint32_t)((size_t)k * a.N + n);
    S.q[0].x = ld4(rw, ok ? base : kOOB);
    S.q[0].y = ld4(rw, ok ? base + a.N : kOOB);
    S.q[0].z = ld4(rw, ok ? base + 2 * a.N : kOOB);
    S.q[0].w = ld4(rw, ok ? base + 3 * a.N : kOOB);
    S.q[1].x = ld4(rw, ok ? base + 4 * a.N : kOOB);
    S.q[1].y = ld4(rw, ok ? base + 5 * a.N : kOOB);
    S.q[1].z = ld4(rw, ok ? base + 6 * a.N : kOOB);
    S.q[1].w = ld4(rw, ok ? base + 7 * a.N : kOOB);
    S.s = ld8(rs, so);
  } else if constexpr (WF == W_I8_NK) {
    // 4 columns (rows of [N, K]) x 8 k bytes each
    const uint32_t base = (uint32_t)((size_t)n * a.K + k);
    uint2 r0 = ld8(rw, ok ? base : kOOB), r1 = ld8(rw, ok ? base + a.K : kOOB);
    uint2 r2 = ld8(rw, ok ? base + 2 * a.K : kOOB), r3 = ld8(rw, ok ? base + 3 * a.K : kOOB);
    S.q[0] = make_uint4(r0.x, r0.y, r1.x, r1.y);
    S.q[1] = make_uint4(r2.x, r2.y, r3.x, r3.y);
    S.s = ld8(rs, so);
  } else if constexpr (WF == W_DENSE_KN) {
    // 8 rows k x 4 columns of T: 8 x 8 bytes
    const uint32_t base = (uint32_t)(((size_t)k * a.N + n) * 2);
    uint2 r[8];
#pragma unroll
    for (int i = 0; i < 8; i++) r[i] = ld8(rw, ok ? base + (uint32_t)(i * a.N * 2) : kOOB);
    S.q[0] = make_uint4(r[0].x, r[0].y, r[1].x, r[1].y);
    S.q[1] = make_uint4(r[2].x, r[2].y, r[3].x, r[3].y);
    S.d[0] = make_uint4(r[4].x, r[4].y, r[5].x, r[5].y);
    S.d[1] = make_uint4(r[6].x, r[6].y, r[7].x, r[7].y);
  } else if constexpr (is_gguf(WF)) {
    // GGUF SoA [N, K] (reference layout: all block headers, then all
    // payloads); 4 weight rows n..n+3 x 8 k.  Raw words only: the header
    // half / sub-block selectors depend on indices, not on the loaded data.
    constexpr int BE = WF == W_Q4K ? 256 : 32;                     // elements per block
    constexpr int HB = WF == W_Q4K ? 16 : 2;                       // header bytes
    constexpr int PB = WF == W_Q4K ? 128 : WF == W_Q80 ? 32 : 16;  // payload bytes
    const int nbr = a.K / BE;
    const uint32_t codes_at = (uint32_t)((size_t)a.N * nbr * HB);
    const int e = k % BE;
    // payload byte of element e's 8-run: Q8_0 e; Q4_0 e % 16 (nibble half
    // e / 16); Q4_K 32 (e / 64) + e % 32 (nibble half (e / 32) % 2)
    const int pb = WF == W_Q80 ? e : WF == W_Q40 ? (e & 15) : 32 * (e >> 6) + (e & 31);
    uint2 r[4];
    uint32_t sel = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const size_t b = (size_t)(n + j) * nbr + (k < a.K ? k : 0) / BE;
      r[j] = ld8(rw, ok ? codes_at + (uint32_t)(b * PB + pb) : kOOB);
      if constexpr (WF == W_Q4K) {
        S.h[j] = ld16(rw, ok ? (uint32_t)(b * 16) : kOOB);
      } else {
        const uint32_t hw = ld4(rw, ok ? (uint32_t)((b * 2) & ~(size_t)3) : kOOB);
        if (j == 0) S.h[0].x = hw;
        else if (j == 1) S.h[0].y = hw;
        else if (j == 2) S.h[0].z = hw;
        else S.h[0].w = hw;
        sel |= (uint32_t)(b & 1) << j;  // d in the high half of its dword
      }
    }
    S.q[0] = make_uint4(r[0].x, r[0].y, r[1].x, r[1].y);
    S.q[1] = make_uint4(r[2].x, r[2].y, r[3].x, r[3].y);
    // Q4_K: sub-block e / 32 and nibble half; Q4_0: nibble half
    S.z.y = WF == W_Q4K ? (uint32_t)(e >> 5) | ((uint32_t)((e >> 5) & 1) << 3)
                        : (uint32_t)(e >> 4);
    S.z.x = sel;
  } else {  // W_DENSE_NK: 4 columns x 8 k of T = 4 x 16 bytes
    const uint32_t base = (uint32_t)(((size_t)n * a.K + k) * 2);
    S.q[0] = ld16(rw, ok ? base : kOOB);
    S.q[1] = ld16(rw, ok ? base + (uint32_t)(a.K * 2) : kOOB);
    S.d[0] = ld16(rw, ok ? base + (uint32_t)(2 * a.K * 2) : kOOB);
    S.d[1] = ld16(rw, ok ? base + (uint32_t)(3 * a.K * 2) : kOOB);
  }
}

__device__ __forceinline__ uint32_t word(const uint4& v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}
__device__ __forceinline__ uint32_t half16(const uint2& v, int j) {
  const uint32_t w = j < 2 ? v.x : v.y;
  return (j & 1) ? (w >> 16) : (w & 0xffff);
}

// Turn the slab into 4 columns x 8 k of T and store them as Bs[n][k..k+7].
template <int WF, int DT>
__device__ __forceinline__ void store_slab(const Slab& S, uint16_t* Bs, int k8, int c,
                                           size_t ldb = LDK) {
  uint32_t out[4][4];  // [column][k pair]
  if constexpr (WF == W_GPTQ4) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t qw = word(S.q[0], j);
      const float s = tof<DT>(half16(S.s, j));
      const int z = (S.z.x >> (4 * ((4 * c + j) & 7))) & 15;
      const float zs = (float)z * s;  // exact: <= 4-bit x T
#pragma unroll
      for (int p = 0; p < 4; p++) {
        // q*s and z*s are exact in f32, so fma(q, s, -z*s) = (q - z) * s exactly
        const float lo = __builtin_fmaf((float)((qw >> (8 * p)) & 15), s, -zs);
        const float hi = __builtin_fmaf((float)((qw >> (8 * p + 4)) & 15), s, -zs);
        out[j][p] = pack2<DT>(lo, hi);
      }
    }
  } else if constexpr (WF == W_U4REF) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float s = tof<DT>(half16(S.s, j)), z = tof<DT>(half16(S.z, j));
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const uint32_t byte = (word(S.q[0], p) >> (8 * j)) & 0xff;  // row k/2+p, column j
        const float lo = __fmul_rn(__fsub_rn((float)(byte & 15), z), s);
        const float hi = __fmul_rn(__fsub_rn((float)(byte >> 4), z), s);
        out[j][p] = pack2<DT>(lo, hi);
      }
    }
  } else if constexpr (WF == W_I8_KN) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float s = tof<DT>(half16(S.s, j));
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const uint32_t w0 = p < 2 ? word(S.q[0], 2 * p) : word(S.q[1], 2 * p - 4);
        const uint32_t w1 = p < 2 ? word(S.q[0], 2 * p + 1) : word(S.q[1], 2 * p - 3);
        const float lo = (float)(int8_t)((w0 >> (8 * j)) & 0xff) * s;
        const float hi = (float)(int8_t)((w1 >> (8 * j)) & 0xff) * s;
        out[j][p] = pack2<DT>(lo, hi);
      }
    }
  } else if constexpr (WF == W_I8_NK) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float s = tof<DT>(half16(S.s, j));
      const uint4& src = j < 2 ? S.q[0] : S.q[1];
      const uint32_t wa = word(src, 2 * (j & 1)), wb = word(src, 2 * (j & 1) + 1);
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const uint32_t w = p < 2 ? wa : wb;
        const int sh = 16 * (p & 1);
        const float lo = (float)(int8_t)((w >> sh) & 0xff) * s;
        const float hi = (float)(int8_t)((w >> (sh + 8)) & 0xff) * s;
        out[j][p] = pack2<DT>(lo, hi);
      }
    }
  } else if constexpr (is_gguf(WF)) {
    // the dequantized values of dequantize_block_* (exact in f32, one rounding to T)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint4& src = j < 2 ? S.q[0] : S.q[1];
      const uint32_t w0 = word(src, 2 * (j & 1)), w1 = word(src, 2 * (j & 1) + 1);
      float mul, sub = 0.f;
      int shift = 0;
      if constexpr (WF == W_Q4K) {
        const uint4 hd = S.h[j];
        int sc, mn;
        q4k_scale_min((int)(S.z.y & 7), hd.y, hd.z, hd.w, sc, mn);
        mul = ub_f16_to_f32((uint16_t)(hd.x & 0xffff)) * (float)sc;
        sub = ub_f16_to_f32((uint16_t)(hd.x >> 16)) * (float)mn;
        shift = 4 * (int)(S.z.y >> 3);
      } else {
        const uint32_t hw = word(S.h[0], j);
        mul = ub_f16_to_f32((uint16_t)(((S.z.x >> j) & 1) ? hw >> 16 : hw & 0xffff));
        // Q8_0 to bf16 rounds the scale to bf16 first (quant.cpp:250), as
        // dequantize_block_q8_0_bf16 does
        if constexpr (WF == W_Q80 && DT == UB_BF16) mul = tof<DT>(ub_f32_to_bf16(mul));
        shift = WF == W_Q40 ? 4 * (int)S.z.y : 0;
      }
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const uint32_t w = p < 2 ? w0 : w1;
        float v[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
          const uint32_t byte = (w >> (16 * (p & 1) + 8 * t)) & 0xff;
          if constexpr (WF == W_Q80) v[t] = mul * (float)(int8_t)byte;
          else if constexpr (WF == W_Q40) v[t] = mul * (float)((int)((byte >> shift) & 15) - 8);
          else v[t] = mul * (float)((byte >> shift) & 15) - sub;
        }
        out[j][p] = pack2<DT>(v[0], v[1]);
      }
    }
  } else if constexpr (WF == W_DENSE_KN) {
    // rows: r0..r3 in q[0], q[1]; r4..r7 in d[0], d[1]; each row = 4 columns (2 words)
    uint2 r[8] = {make_uint2(S.q[0].x, S.q[0].y), make_uint2(S.q[0].z, S.q[0].w),
                  make_uint2(S.q[1].x, S.q[1].y), make_uint2(S.q[1].z, S.q[1].w),
                  make_uint2(S.d[0].x, S.d[0].y), make_uint2(S.d[0].z, S.d[0].w),
                  make_uint2(S.d[1].x, S.d[1].y), make_uint2(S.d[1].z, S.d[1].w)};
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int p = 0; p < 4; p++)
        out[j][p] = half16(r[2 * p], j) | (half16(r[2 * p + 1], j) << 16);
  } else {
    const uint4 cols[4] = {S.q[0], S.q[1], S.d[0], S.d[1]};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      out[j][0] = cols[j].x;
      out[j][1] = cols[j].y;
      out[j][2] = cols[j].z;
      out[j][3] = cols[j].w;
    }
  }
#pragma unroll
  for (int j = 0; j < 4; j++)
    *(uint4*)(Bs + (size_t)(4 * c + j) * ldb + 8 * k8) =
        make_uint4(out[j][0], out[j][1], out[j][2], out[j][3]);
}

template <int DT>
__device__ __forceinline__ f32x16 mfma(const uint4& a, const uint4& b, const f32x16& c) {
  if constexpr (DT == UB_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Block tile BM x BN (4 wavefronts in 2 x 2, each (BM/2) x (BN/2) = TM x TN
// MFMA 32x32 tiles).  256 x 256 halves the LDS bytes per flop of 128 x 128
// and gives each K-step ~4x the MFMA time to hide the next step's loads.
template <int WF, int DT, int BM, int BN>
__global__ void __launch_bounds__(256, BM * BN >= 256 * 256 ? 1 : 2)
    __attribute__((amdgpu_waves_per_eu(BM * BN >= 256 * 256 ? 1 : 2, BM * BN >= 256 * 256 ? 1 : 2)))
    k_gemm(GemmArgs a) {
  constexpr int TM = BM / 64, TN = BN / 64;  // 32x32 MFMA tiles per wavefront
  constexpr int AQ = BM / 32;                // 16-byte A chunks per thread per K-step
  constexpr int NS = BN / 128;               // weight slabs per thread per K-step
  __shared__ __align__(16) uint16_t As[2][BM * LDK];
  __shared__ __align__(16) uint16_t Bs[2][BN * LDK];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM, b = blockIdx.z;

  const uint16_t* A = (const uint16_t*)a.a + (size_t)b * a.sa;
  const __amdgpu_buffer_rsrc_t ra = rsrc(A, (uint64_t)a.M * a.K * 2);
  const uint8_t* W = (const uint8_t*)a.w + (size_t)b * a.sw;
  uint64_t wbytes;
  if constexpr (WF == W_GPTQ4) wbytes = (uint64_t)a.K / 8 * a.N * 4;
  else if constexpr (WF == W_U4REF) wbytes = (uint64_t)a.K / 2 * a.N;
  else if constexpr (WF == W_I8_KN || WF == W_I8_NK) wbytes = (uint64_t)a.K * a.N;
  else if constexpr (WF == W_Q4K) wbytes = (uint64_t)a.K / 256 * a.N * 144;
  else if constexpr (WF == W_Q80) wbytes = (uint64_t)a.K / 32 * a.N * 34;
  else if constexpr (WF == W_Q40) wbytes = (uint64_t)a.K / 32 * a.N * 18;
  else wbytes = (uint64_t)a.K * a.N * 2;
  const __amdgpu_buffer_rsrc_t rw = rsrc(W, wbytes);
  const int ng = (a.K + a.group - 1) / a.group;
  const __amdgpu_buffer_rsrc_t rs = rsrc(a.scales, (uint64_t)ng * a.N * 2);
  const __amdgpu_buffer_rsrc_t rz =
      rsrc(a.zeros, WF == W_GPTQ4 ? (uint64_t)ng * (a.N / 8) * 4 : (uint64_t)ng * a.N * 2);

  // Global -> register staging of one K-step (A chunks and weight slabs).
  // A: BM rows x 8 chunks of 8 elements; chunk q = tid + 256 i -> row q/8.
  // Weight slabs: (k8 = tid/32, c = tid%32 + 32 j), j < NS.  Loads past K
  // read zero, so the staging runs unconditionally (no branch joins).
  uint4 ar[1][AQ];
  Slab S[1][NS];
  const int k8 = tid >> 5;
  auto load_ab = [&](int st, int k0) {
#pragma unroll
    for (int i = 0; i < AQ; i++) {
      const int q = tid + 256 * i;
      const int m = m0 + (q >> 3), k = k0 + 8 * (q & 7);
      const bool ok = m < a.M && k < a.K;
      ar[st][i] = ld16(ra, ok ? (uint32_t)(((size_t)m * a.K + k) * 2) : kOOB);
    }
#pragma unroll
    for (int j = 0; j < NS; j++)
      load_slab<WF, DT>(S[st][j], a, rw, rs, rz, k0, n0, k8, (tid & 31) + 32 * j);
  };
  auto store_ab = [&](int st, int buf) {
#pragma unroll
    for (int i = 0; i < AQ; i++) {
      const int q = tid + 256 * i;
      *(uint4*)(As[buf] + (size_t)(q >> 3) * LDK + 8 * (q & 7)) = ar[st][i];
    }
#pragma unroll
    for (int j = 0; j < NS; j++) store_slab<WF, DT>(S[st][j], Bs[buf], k8, (tid & 31) + 32 * j);
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  const int l32 = lane & 31, kh = lane >> 5;
  auto compute = [&](int cur) {
    const uint16_t* Ac = As[cur] + (size_t)(wm * (BM / 2) + l32) * LDK + 8 * kh;
    const uint16_t* Bc = Bs[cur] + (size_t)(wn * (BN / 2) + l32) * LDK + 8 * kh;
    // fragments double-buffered across the four 16-k substeps: the LDS reads
    // of substep kk+1 are in flight while substep kk's MFMAs run
    uint4 af[2][TM], bfr[2][TN];
#pragma unroll
    for (int i = 0; i < TM; i++) af[0][i] = *(const uint4*)(Ac + (size_t)i * 32 * LDK);
#pragma unroll
    for (int j = 0; j < TN; j++) bfr[0][j] = *(const uint4*)(Bc + (size_t)j * 32 * LDK);
#pragma unroll
    for (int kk = 0; kk < BK / 16; kk++) {
      const int fc = kk & 1, fn = fc ^ 1;
      if (kk + 1 < BK / 16) {
#pragma unroll
        for (int i = 0; i < TM; i++)
          af[fn][i] = *(const uint4*)(Ac + (size_t)i * 32 * LDK + (kk + 1) * 16);
#pragma unroll
        for (int j = 0; j < TN; j++)
          bfr[fn][j] = *(const uint4*)(Bc + (size_t)j * 32 * LDK + (kk + 1) * 16);
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = mfma<DT>(af[fc][i], bfr[fc][j], acc[i][j]);
      // interleave: one LDS fragment read between consecutive MFMAs
#pragma unroll
      for (int q = 0; q < TM * TN; q++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 DS read
      }
    }
  };

  // One register stage: step kt+1 is loaded while step kt's MFMAs run, then
  // stored to the other LDS buffer.  (A second register stage spills the
  // 256 x 256 tile and measured slower on the smaller tiles.)
  const int nk = (a.K + BK - 1) / BK;
  load_ab(0, 0);
  store_ab(0, 0);
  __syncthreads();
  for (int kt = 0; kt < nk; kt++) {
    const int cur = kt & 1;
    load_ab(0, (kt + 1) * BK);  // past the end of K these read zero
    compute(cur);
    store_ab(0, cur ^ 1);
    __syncthreads();
  }

  // epilogue: lane l, register r of block (i, j) holds
  // C[m0 + wm*BM/2 + 32i + 8(r/4) + 4(l/32) + r%4][n0 + wn*BN/2 + 32j + l%32]
  uint16_t* C = (uint16_t*)a.c + (size_t)b * a.sc * (a.c_f32 ? 2 : 1);
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int n = n0 + wn * (BN / 2) + 32 * j + l32;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int m = m0 + wm * (BM / 2) + 32 * i + 8 * (r >> 2) + 4 * kh + (r & 3);
        if (m < a.M && n < a.N) {
          const float v = acc[i][j][r];
          if (a.c_f32) ((float*)C)[(size_t)m * a.N + n] = v;
          else C[(size_t)m * a.N + n] = (uint16_t)(pack2<DT>(v, 0.f) & 0xffff);
        }
      }
    }
}

// The dequantized weight of columns [n0, n0 + nc) as a T slab out[nc, K]
// (column-major: row j = column n0 + j, k contiguous), the values the MFMA
// core produces into LDS.  One thread per 4-column x 8-k slab; a block holds
// kDeqCG(WF) neighbouring 4-column groups x 256 / kDeqCG(WF) k8 steps, so
// that a wave reads 64 contiguous bytes of a [K, N]-major weight row and
// writes 256 contiguous bytes of each slab row (k-fastest alone for [N, K]).
template <int WF>
constexpr int kDeqCG = WF == W_I8_NK ? 1 : 4;
template <int WF, int DT>
__global__ void __launch_bounds__(256) k_deq_nk(GemmArgs a, int n0, int nc, uint16_t* out) {
  constexpr int CG = kDeqCG<WF>;
  const int k8n = a.K / 8;
  const int c = blockIdx.y * CG + (int)threadIdx.x % CG;
  const int k8 = blockIdx.x * (256 / CG) + (int)threadIdx.x / CG;
  if (c >= nc / 4 || k8 >= k8n) return;
  const uint8_t* W = (const uint8_t*)a.w;
  uint64_t wbytes;
  if constexpr (WF == W_GPTQ4) wbytes = (uint64_t)a.K / 8 * a.N * 4;
  else if constexpr (WF == W_U4REF) wbytes = (uint64_t)a.K / 2 * a.N;
  else wbytes = (uint64_t)a.K * a.N;
  const __amdgpu_buffer_rsrc_t rw = rsrc(W, wbytes);
  const int ng = (a.K + a.group - 1) / a.group;
  const __amdgpu_buffer_rsrc_t rs = rsrc(a.scales, (uint64_t)ng * a.N * 2);
  const __amdgpu_buffer_rsrc_t rz =
      rsrc(a.zeros, WF == W_GPTQ4 ? (uint64_t)ng * (a.N / 8) * 4 : (uint64_t)ng * a.N * 2);
  Slab S;
  load_slab<WF, DT>(S, a, rw, rs, rz, 0, n0, k8, c);
  store_slab<WF, DT>(S, out, k8, c, (size_t)a.K);
}

template <int WF, int DT, int BM, int BN>
int launch_tile(const GemmArgs& a, int batch, hipStream_t s) {
  dim3 grid(ub_cdiv(a.N, BN), ub_cdiv(a.M, BM), batch);
  k_gemm<WF, DT, BM, BN><<<grid, 256, 0, s>>>(a);
  return ub_check_launch("gemm");
}

// Tile choice: 256 x 256 once there are enough tiles of that size to fill the
// CUs, 128 x 128 otherwise (128 x 256 measured slower than both); the
// gemm_tile knob overrides.  Returns 1 (128 x 128), 2 (128 x 256) or 3 (256 x 256).
int plan_tile(long M, long N, long batch) {
  const long tiles256 = ub_cdiv(N, 256) * ub_cdiv(M, 256) * batch;
  const int t = ub_tune(UB_TUNE_GEMM_TILE);
  if (t >= 1 && t <= 3) return t;
  return tiles256 >= 384 ? 3 : 1;
}
// The tile a (sip_m, sip_n) pair names, 0 if none (then the shape rule decides).
int tile_of(int sip_m, int sip_n) {
  if (sip_m == 128 && sip_n == 128) return 1;
  if (sip_m == 128 && sip_n == 256) return 2;
  if (sip_m == 256 && sip_n == 256) return 3;
  return 0;
}

template <int WF, int DT>
int launch(const GemmArgs& a, int batch, hipStream_t s, int tile) {
  const int t = tile ? tile : plan_tile(a.M, a.N, batch);
  if (t == 3) return launch_tile<WF, DT, 256, 256>(a, batch, s);
  if (t == 2) return launch_tile<WF, DT, 128, 256>(a, batch, s);
  return launch_tile<WF, DT, 128, 128>(a, batch, s);
}

int gemm_dispatch(int wf, int dt, const GemmArgs& a, int batch, hipStream_t s, int tile = 0) {
#define UB_G(WF)                                           \
  if (wf == WF) return dt == UB_BF16 ? launch<WF, UB_BF16>(a, batch, s, tile) \
                                     : launch<WF, UB_F16>(a, batch, s, tile);
  UB_G(W_GPTQ4) UB_G(W_U4REF) UB_G(W_I8_KN) UB_G(W_I8_NK) UB_G(W_DENSE_KN) UB_G(W_DENSE_NK)
  if (dt == UB_BF16) {  // GGUF weights: bf16 activations only
    if (wf == W_Q40) return launch<W_Q40, UB_BF16>(a, batch, s, tile);
    if (wf == W_Q80) return launch<W_Q80, UB_BF16>(a, batch, s, tile);
    if (wf == W_Q4K) return launch<W_Q4K, UB_BF16>(a, batch, s, tile);
  }
#undef UB_G
  return ub_set_error(UB_ERR_UNSUPPORTED, "gemm: weight format %d", wf);
}

// Quantized weights at large M: the weight dequantized once, in column slabs
// of up to 256 MB of T, into the per-stream library workspace, each slab a
// hipBLASLt GEMM.  The fused kernels dequantize every weight once per M tile,
// which at these M costs more than one dequantization pass plus a dense GEMM.
// MI355X, 4096 x 14336 (us, slab route / pipelined kernel): GPTQ 512 75.7 /
// 62.7, 1024 111.1 / 108.3, 1280 151.1 / 185.5, 2048 193 / 227; uint8 4-bit
// 512 78.8 / 72.8, 768 102.5 / 115.8, 1024 114.7 / 123.6, 1280 154.3 / 218.0;
// int8 [N,K] 768 104.2 / 101.5, 1024 112.4 / 113.8, 1280 153.9 / 195.9.
// UB_ERR_UNSUPPORTED when it cannot run (hipBLASLt has no algorithm for the
// shape, or the scratch allocation failed); the caller then takes the fused
// kernels.
int lib_min_m(int wf) { return wf == W_U4REF ? 640 : 1025; }
constexpr size_t kLibSlabBytes = 256ull << 20;
int lib_route(int wf, int dt, const GemmArgs& ga, int M, hipStream_t s) {
  const int N = ga.N, K = ga.K;
  const int path = ub_tune(UB_TUNE_W4A16_PATH);  // 6: this route from 17 tokens
  if ((wf != W_GPTQ4 && wf != W_U4REF && wf != W_I8_KN && wf != W_I8_NK) ||
      (path == 6 ? M <= 16 : path != 0 || M < lib_min_m(wf)))
    return UB_ERR_UNSUPPORTED;
  int nc = (int)std::min<size_t>((size_t)N, std::max<size_t>(256, kLibSlabBytes / ((size_t)K * 2)));
  nc -= nc % 4;
  const int tail = N % nc;
  if (!ub_blaslt_ready(1, M, nc, K, 1, 0, N, 0, dt, s) ||
      (tail && !ub_blaslt_ready(1, M, tail, K, 1, 0, N, 0, dt, s)))
    return UB_ERR_UNSUPPORTED;
  UbScratch ws(s, (size_t)nc * K * 2);
  uint16_t* slab = (uint16_t*)ws.get();
  if (!slab) return UB_ERR_UNSUPPORTED;
  for (int n0 = 0; n0 < N; n0 += nc) {
    const int w = std::min(nc, N - n0);
#define UB_DQ(WF)                                                                 \
    if (wf == WF) {                                                               \
      const dim3 g(ub_cdiv(K / 8, 256 / kDeqCG<WF>), ub_cdiv(w / 4, kDeqCG<WF>)); \
      if (dt == UB_BF16) k_deq_nk<WF, UB_BF16><<<g, 256, 0, s>>>(ga, n0, w, slab); \
      else k_deq_nk<WF, UB_F16><<<g, 256, 0, s>>>(ga, n0, w, slab);              \
    }
    UB_DQ(W_GPTQ4) UB_DQ(W_U4REF) UB_DQ(W_I8_KN) UB_DQ(W_I8_NK)
#undef UB_DQ
    const int e = ub_blaslt_gemm(ga.a, slab, (uint16_t*)ga.c + n0, 1, M, w, K, 1, 0, N, 0, dt, s);
    if (e) return ub_set_error(e == UB_ERR_UNSUPPORTED ? UB_ERR_LAUNCH : e,
                               "quantized GEMM: library GEMM of a slab failed");
  }
  return ub_check_launch("quantized GEMM (slab route)");
}

int check_shape(const char* nm, int M, int N, int K, int group, int wf) {
  UB_REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative shape", nm);
  UB_REQUIRE(K % 8 == 0, "%s: K=%d must be a multiple of 8", nm, K);
  UB_REQUIRE(N % (wf == W_GPTQ4 ? 8 : 4) == 0, "%s: N=%d must be a multiple of %d", nm, N,
             wf == W_GPTQ4 ? 8 : 4);
  UB_REQUIRE(group > 0 && group % 8 == 0, "%s: group size %d must be a positive multiple of 8",
             nm, group);
  return UB_OK;
}

// The GEMM routes read A rows with 16-byte loads.  An A that is not 16-byte
// aligned (a view into a larger tensor) is copied once into call scratch and
// the copy is used instead; `a` stays as given otherwise.
struct AlignedA {
  UbScratch ws;
  const void* a;
  int err = UB_OK;
  AlignedA(const void* a0, size_t elems, hipStream_t s)
      : ws(s, ((uintptr_t)a0 & 15) ? elems * 2 : 0), a(a0) {
    if (((uintptr_t)a0 & 15) == 0) return;
    if (!ws.get()) {
      err = ub_set_error(UB_ERR_LAUNCH, "could not allocate %zu bytes to align A", elems * 2);
      return;
    }
    err = ub_copy_b16(a0, ws.get(), elems, s);
    a = ws.get();
  }
};

// Reference matmul_* argument block (kernels/matmul.cpp:1143-1215).
struct RefMM {
  int input_dtype, batch, m, k, n, lhs_mc, rhs_mc, batch_mc, lhs_t, rhs_t;
  float alpha, beta, addmm_beta;
  int sip_m, sip_k, sip_n, broadcasted_weight;
};

int ref_matmul(const char* nm, int wf, int dt, const void* a, const void* b, void* out,
               const void* scales, const void* zeros, const RefMM& r, int group, void* stream) {
  UB_REQUIRE(r.lhs_t == 0, "%s: lhs_transpose is not supported", nm);
  UB_REQUIRE(r.batch >= 1 || r.m * r.n == 0, "%s: batch %d", nm, r.batch);
  // Tiling hints: a (sip_m, sip_n) pair naming one of this library's tiles
  // (what ubridge_get_gemm_launch_params hands out) selects it; anything else
  // (e.g. zeros, or GCU tilings) leaves the choice to the shape rule.
  // sip_k and the *_multicore flags are informational.
  const int g = group <= 0 ? r.k : group;
  int e = check_shape(nm, r.m, r.n, r.k, g, wf);
  if (e) return e;
  if ((size_t)r.m * r.n * r.batch == 0) return UB_OK;
  UB_REQUIRE(a && b && out, "%s: null pointer", nm);
  ub_blaslt_prepare(ub_stream(stream));
  AlignedA al(a, (size_t)r.m * r.batch * r.k, ub_stream(stream));
  if (al.err) return al.err;
  a = al.a;
  GemmArgs ga{};
  ga.a = a;
  ga.w = b;
  ga.scales = scales;
  ga.zeros = zeros;
  ga.c = out;
  ga.M = r.m;
  ga.N = r.n;
  ga.K = r.k;
  ga.group = g;
  ga.sa = (long long)r.m * r.k;
  ga.sc = (long long)r.m * r.n;
  long long wb;
  if (wf == W_U4REF) wb = (long long)r.k / 2 * r.n;
  else if (wf == W_I8_KN || wf == W_I8_NK) wb = (long long)r.k * r.n;
  else wb = (long long)r.k * r.n * 2;
  ga.sw = r.broadcasted_weight > 0 ? 0 : wb;
  UB_REQUIRE(r.broadcasted_weight > 0 || r.batch == 1 || wf >= W_DENSE_KN,
             "%s: per-batch quantized weights need per-batch scales; pass broadcasted_weight=1",
             nm);
  // Dense weights at up to 16 tokens (one weight for every batch): the decode
  // GEMV, which streams the weight with every CU instead of one workgroup per
  // 128 output columns (knob w4a16_path: 2 skips it, 1 also the library GEMM
  // below, for this file's MFMA core)
  if ((wf == W_DENSE_KN || wf == W_DENSE_NK) && (r.broadcasted_weight > 0 || r.batch == 1) &&
      ub_tune(UB_TUNE_W4A16_PATH) != 2 && ub_tune(UB_TUNE_W4A16_PATH) != 1) {
    const int e1 = ub_wq_gemv(wf, a, b, nullptr, nullptr, out, r.m * r.batch, r.k, r.n, r.k, dt,
                              ub_stream(stream));
    if (e1 != UB_ERR_UNSUPPORTED) return e1;
  }
  // Dense weights otherwise: a plain library GEMM (hipBLASLt), unless the
  // w4a16_path = 1 knob asks for this file's MFMA core
  if ((wf == W_DENSE_KN || wf == W_DENSE_NK) && ub_tune(UB_TUNE_W4A16_PATH) != 1) {
    const int e1 = ub_blaslt_gemm(a, b, out, r.batch, r.m, r.n, r.k, wf == W_DENSE_NK,
                                  r.broadcasted_weight > 0, r.n, 0, dt, ub_stream(stream));
    if (e1 != UB_ERR_UNSUPPORTED) return e1;
  }
  // Quantized formats: the pipelined kernel of w4a16.hip (one weight for
  // every batch, so the batches fold into M); shapes outside its contract
  // and the w4a16_path = 1 knob take this file's MFMA core.
  if (wf >= W_U4REF && wf <= W_I8_NK && ub_tune(UB_TUNE_W4A16_PATH) != 1) {
    if (ub_tune(UB_TUNE_W4A16_PATH) != 2) {  // up to 16 tokens: the decode GEMV
      const int e1 = ub_wq_gemv(wf, a, b, scales, zeros, out, r.m * r.batch, r.k, r.n, g, dt,
                                ub_stream(stream));
      if (e1 != UB_ERR_UNSUPPORTED) return e1;
    }
    if (r.broadcasted_weight > 0 || r.batch == 1) {  // large M: dequantized slabs + hipBLASLt
      GemmArgs gl = ga;
      gl.M = r.m * r.batch;
      const int e1 = lib_route(wf, dt, gl, gl.M, ub_stream(stream));
      if (e1 != UB_ERR_UNSUPPORTED) return e1;
    }
    const int t = tile_of(r.sip_m, r.sip_n);
    const int e2 = ub_wq_pipelined(wf, a, b, scales, zeros, out, r.m * r.batch, r.k, r.n, g, dt,
                                   t == 2 ? 1 : t == 3 ? 2 : 0, ub_stream(stream));
    if (e2 != UB_ERR_UNSUPPORTED) return e2;
  }
  return gemm_dispatch(wf, dt, ga, r.batch, ub_stream(stream), tile_of(r.sip_m, r.sip_n));
}

}  // namespace

// =================================================================== ABI
int ub_w4a16_pipelined(const void* a, const int32_t* qw, const void* scales, const int32_t* qzeros,
                       void* out, int M, int K, int N, int group, int dtype, hipStream_t s);

// North-star W4A16 (GPTQ-style layout): out[M,N] = a[M,K] . deq(qw)[K,N].
// Up to 16 tokens the decode GEMV; beyond 1024 tokens the weight dequantized
// in slabs and hipBLASLt; between, group sizes and K that are multiples of 64
// take the pipelined kernel of w4a16.hip; the rest (and the w4a16_path = 1
// knob) this file's MFMA core.
UB_API int ubridge_w4a16_gemm(const void* a, const int32_t* qw, const void* scales,
                              const int32_t* qzeros, void* out, int M, int K, int N, int group,
                              int dtype, void* stream) {
  const char* nm = "ubridge_w4a16_gemm";
  int e = check_shape(nm, M, N, K, group, W_GPTQ4);
  if (e) return e;
  UB_REQUIRE(dtype == UB_BF16 || dtype == UB_F16, "%s: dtype %d (f16=1, bf16=2)", nm, dtype);
  if ((size_t)M * N == 0) return UB_OK;
  UB_REQUIRE(a && qw && scales && qzeros && out, "%s: null pointer", nm);
  ub_blaslt_prepare(ub_stream(stream));
  AlignedA al(a, (size_t)M * K, ub_stream(stream));
  if (al.err) return al.err;
  a = al.a;
  if (ub_tune(UB_TUNE_W4A16_PATH) != 1) {
    if (ub_tune(UB_TUNE_W4A16_PATH) != 2) {  // up to 16 tokens: the decode GEMV
      const int e1 = ub_wq_gemv(W_GPTQ4, a, qw, scales, qzeros, out, M, K, N, group, dtype,
                                ub_stream(stream));
      if (e1 != UB_ERR_UNSUPPORTED) return e1;
    }
    {  // beyond 1024 tokens: dequantized slabs + hipBLASLt
      GemmArgs gl{a, qw, scales, qzeros, out, M, N, K, group, 0, 0, 0};
      const int e1 = lib_route(W_GPTQ4, dtype, gl, M, ub_stream(stream));
      if (e1 != UB_ERR_UNSUPPORTED) return e1;
    }
    const int e2 = ub_w4a16_pipelined(a, qw, scales, qzeros, out, M, K, N, group, dtype,
                                      ub_stream(stream));
    if (e2 != UB_ERR_UNSUPPORTED) return e2;
  }
  GemmArgs ga{a, qw, scales, qzeros, out, M, N, K, group, 0, 0, 0};
  return gemm_dispatch(W_GPTQ4, dtype, ga, 1, ub_stream(stream));
}

// Dense weight GEMM on the same core: w [K,N] (w_transposed = 0) or [N,K].
// y[M, N] = x[M, K] . deq(W)[N, K]^T for a GGUF SoA weight (qtype 2 Q4_0,
// 8 Q8_0, 12 Q4_K), x bf16, y f32 (y_f32) or bf16: the dequantize_block_* values
// produced tile by tile into LDS, never in HBM.  UB_ERR_UNSUPPORTED (nothing
// recorded) outside K % block == 0, N % 4 == 0, weight below 2 GiB.
int ub_gguf_gemm(int qtype, const void* w, const void* x, void* y, int y_f32, int M, int N, int K,
                 hipStream_t s) {
  const int be = qtype == UB_Q4_K ? 256 : 32;
  const int wf = qtype == UB_Q4_K ? W_Q4K : qtype == UB_Q8_0 ? W_Q80 : qtype == UB_Q4_0 ? W_Q40 : -1;
  const size_t wb = (size_t)N * K / be * (qtype == UB_Q4_K ? 144 : qtype == UB_Q8_0 ? 34 : 18);
  if (wf < 0 || M < 1 || N < 1 || K < be || K % be || N % 4 || wb >= 0x80000000ull ||
      (size_t)M * K * 2 >= 0x80000000ull)
    return UB_ERR_UNSUPPORTED;
  GemmArgs ga{x, w, nullptr, nullptr, y, M, N, K, be, 0, 0, 0, y_f32};
  return gemm_dispatch(wf, UB_BF16, ga, 1, s);
}

UB_API int ubridge_gemm_dense(const void* a, const void* w, void* out, int M, int K, int N,
                              int w_transposed, int dtype, void* stream) {
  const char* nm = "ubridge_gemm_dense";
  const int wf = w_transposed ? W_DENSE_NK : W_DENSE_KN;
  int e = check_shape(nm, M, N, K, 8, wf);
  if (e) return e;
  if ((size_t)M * N == 0) return UB_OK;
  UB_REQUIRE(a && w && out, "%s: null pointer", nm);
  GemmArgs ga{a, w, nullptr, nullptr, out, M, N, K, 8, 0, 0, 0};
  return gemm_dispatch(wf, dtype, ga, 1, ub_stream(stream));
}

#define UB_REF_ARGS                                                                        \
  int input_dtype, int batch, int m, int k, int n, int lhs_mc, int rhs_mc, int batch_mc,   \
      int lhs_t, int rhs_t, float alpha, float beta, float addmm_beta, int sip_m, int sip_k, \
      int sip_n, int broadcasted_weight
#define UB_REF_PACK                                                                       \
  RefMM r{input_dtype, batch, m, k, n, lhs_mc, rhs_mc, batch_mc, lhs_t, rhs_t, alpha, beta, \
          addmm_beta, sip_m, sip_k, sip_n, broadcasted_weight}

// matmul_{bf16,f16}_4bit (kernels/matmul.cpp:1211-1212): b uint8 [K/2, N].
UB_API void matmul_bf16_4bit(const void* a, const uint8_t* b, void* out, const void* scales,
                             const void* zeros, UB_REF_ARGS, int group_size, void* stream) {
  UB_REF_PACK;
  if (rhs_t) { ub_set_error(UB_ERR_UNSUPPORTED, "matmul_bf16_4bit: rhs_transpose"); return; }
  ref_matmul("matmul_bf16_4bit", W_U4REF, UB_BF16, a, b, out, scales, zeros, r, group_size, stream);
}
UB_API void matmul_f16_4bit(const void* a, const uint8_t* b, void* out, const void* scales,
                            const void* zeros, UB_REF_ARGS, int group_size, void* stream) {
  UB_REF_PACK;
  if (rhs_t) { ub_set_error(UB_ERR_UNSUPPORTED, "matmul_f16_4bit: rhs_transpose"); return; }
  ref_matmul("matmul_f16_4bit", W_U4REF, UB_F16, a, b, out, scales, zeros, r, group_size, stream);
}
// matmul_{bf16,f16}_8bit (kernels/matmul.cpp:1214-1215): b int8 [K, N] or [N, K].
UB_API void matmul_bf16_8bit(const void* a, const int8_t* b, void* out, const void* scales,
                             const void* zeros, UB_REF_ARGS, int group_size, void* stream) {
  UB_REF_PACK;
  (void)zeros;
  ref_matmul("matmul_bf16_8bit", rhs_t ? W_I8_NK : W_I8_KN, UB_BF16, a, b, out, scales, nullptr,
             r, group_size, stream);
}
UB_API void matmul_f16_8bit(const void* a, const int8_t* b, void* out, const void* scales,
                            const void* zeros, UB_REF_ARGS, int group_size, void* stream) {
  UB_REF_PACK;
  (void)zeros;
  ref_matmul("matmul_f16_8bit", rhs_t ? W_I8_NK : W_I8_KN, UB_F16, a, b, out, scales, nullptr, r,
             group_size, stream);
}
// matmul_{bf16,f16} dense (kernels/matmul.cpp:1181-1184).
UB_API void matmul_bf16(const void* a, const void* b, void* out, UB_REF_ARGS, void* stream) {
  UB_REF_PACK;
  ref_matmul("matmul_bf16", rhs_t ? W_DENSE_NK : W_DENSE_KN, UB_BF16, a, b, out, nullptr, nullptr,
             r, 8, stream);
}
UB_API void matmul_f16(const void* a, const void* b, void* out, UB_REF_ARGS, void* stream) {
  UB_REF_PACK;
  ref_matmul("matmul_f16", rhs_t ? W_DENSE_NK : W_DENSE_KN, UB_F16, a, b, out, nullptr, nullptr, r,
             8, stream);
}

// ------------------------------------------------ dequant_{f16,bf16} host lib
// dequant_host.cpp:7-16,298-307: rhs uint8 [K, N] holds 2K weight rows (K is
// the packed row count), scale / zeros T [2K/g, N], out T [2K, N];
// low nibble = row 2k, high nibble = row 2k+1, w = T(((float)q - z) * s).
// One lane per 4 packed bytes (4 columns) -> two 8-byte row stores.
namespace {
template <int DT>
__global__ void __launch_bounds__(256) k_dequant_u4(const uint8_t* __restrict__ rhs,
                                                    const uint16_t* __restrict__ scale,
                                                    const uint16_t* __restrict__ zeros,
                                                    uint16_t* __restrict__ out, int K, int N,
                                                    int group) {
  const size_t n4 = (size_t)N / 4;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < (size_t)K * n4;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t k = i / n4;
    const int n = (int)(i % n4) * 4;
    const uint32_t q = *(const uint32_t*)(rhs + k * N + n);
    const int g0 = (int)(2 * k / group), g1 = (int)((2 * k + 1) / group);
    const uint2 s0 = *(const uint2*)(scale + (size_t)g0 * N + n);
    const uint2 z0 = *(const uint2*)(zeros + (size_t)g0 * N + n);
    const uint2 s1 = *(const uint2*)(scale + (size_t)g1 * N + n);
    const uint2 z1 = *(const uint2*)(zeros + (size_t)g1 * N + n);
    uint32_t lo[2], hi[2];
#pragma unroll
    for (int p = 0; p < 2; p++) {
      float vl[2], vh[2];
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const int j = 2 * p + e;
        const uint32_t byte = (q >> (8 * j)) & 0xff;
        vl[e] = __fmul_rn(__fsub_rn((float)(byte & 15), tof<DT>(half16(z0, j))), tof<DT>(half16(s0, j)));
        vh[e] = __fmul_rn(__fsub_rn((float)(byte >> 4), tof<DT>(half16(z1, j))), tof<DT>(half16(s1, j)));
      }
      lo[p] = pack2<DT>(vl[0], vl[1]);
      hi[p] = pack2<DT>(vh[0], vh[1]);
    }
    *(uint2*)(out + (2 * k) * N + n) = make_uint2(lo[0], lo[1]);
    *(uint2*)(out + (2 * k + 1) * N + n) = make_uint2(hi[0], hi[1]);
  }
}

int dequant_u4(const char* nm, int dt, void* out, const uint8_t* rhs, const void* scale,
               const void* zeros, int K, int N, int weight_transpose, int group, void* stream) {
  if (weight_transpose) return ub_set_error(UB_ERR_UNSUPPORTED, "%s: weight_transpose", nm);
  UB_REQUIRE(K >= 0 && N >= 0 && N % 4 == 0, "%s: K=%d N=%d (N must be a multiple of 4)", nm, K, N);
  if (group <= 0) group = 2 * K;
  UB_REQUIRE(group > 0, "%s: group %d", nm, group);
  if ((size_t)K * N == 0) return UB_OK;
  UB_REQUIRE(out && rhs && scale && zeros, "%s: null pointer", nm);
  size_t work = (size_t)K * N / 4;
  int grid = (int)((work + 255) / 256 < 65536 ? (work + 255) / 256 : 65536);
  hipStream_t s = ub_stream(stream);
  if (dt == UB_BF16)
    k_dequant_u4<UB_BF16><<<grid, 256, 0, s>>>(rhs, (const uint16_t*)scale, (const uint16_t*)zeros,
                                               (uint16_t*)out, K, N, group);
  else
    k_dequant_u4<UB_F16><<<grid, 256, 0, s>>>(rhs, (const uint16_t*)scale, (const uint16_t*)zeros,
                                              (uint16_t*)out, K, N, group);
  return ub_check_launch(nm);
}
}  // namespace

UB_API void dequant_bf16(void* out, const uint8_t* rhs, const void* scale, const void* zeros, int K,
                         int N, int weight_transpose, int group_size, void* stream) {
  dequant_u4("dequant_bf16", UB_BF16, out, rhs, scale, zeros, K, N, weight_transpose, group_size,
             stream);
}
UB_API void dequant_f16(void* out, const uint8_t* rhs, const void* scale, const void* zeros, int K,
                        int N, int weight_transpose, int group_size, void* stream) {
  dequant_u4("dequant_f16", UB_F16, out, rhs, scale, zeros, K, N, weight_transpose, group_size,
             stream);
}

// ------------------------------------------------- name-keyed launch thunks
#define UB_MM_THUNK(NAME, WT)                                                                  \
  void ub_thunk_##NAME(void** args, void* stream) {                                           \
    NAME(UB_ARG(const void*, 0), UB_ARG(const WT*, 1), UB_ARG(void*, 2), UB_ARG(const void*, 3), \
         UB_ARG(const void*, 4), UB_ARG(int, 5), UB_ARG(int, 6), UB_ARG(int, 7), UB_ARG(int, 8), \
         UB_ARG(int, 9), UB_ARG(int, 10), UB_ARG(int, 11), UB_ARG(int, 12), UB_ARG(int, 13),    \
         UB_ARG(int, 14), UB_ARG(float, 15), UB_ARG(float, 16), UB_ARG(float, 17),             \
         UB_ARG(int, 18), UB_ARG(int, 19), UB_ARG(int, 20), UB_ARG(int, 21), UB_ARG(int, 22),   \
         stream);                                                                              \
  }
UB_MM_THUNK(matmul_bf16_4bit, uint8_t)
UB_MM_THUNK(matmul_f16_4bit, uint8_t)
UB_MM_THUNK(matmul_bf16_8bit, int8_t)
UB_MM_THUNK(matmul_f16_8bit, int8_t)
#undef UB_MM_THUNK
#define UB_MMD_THUNK(NAME)                                                                     \
  void ub_thunk_##NAME(void** args, void* stream) {                                           \
    NAME(UB_ARG(const void*, 0), UB_ARG(const void*, 1), UB_ARG(void*, 2), UB_ARG(int, 3),       \
         UB_ARG(int, 4), UB_ARG(int, 5), UB_ARG(int, 6), UB_ARG(int, 7), UB_ARG(int, 8),         \
         UB_ARG(int, 9), UB_ARG(int, 10), UB_ARG(int, 11), UB_ARG(int, 12), UB_ARG(float, 13),   \
         UB_ARG(float, 14), UB_ARG(float, 15), UB_ARG(int, 16), UB_ARG(int, 17), UB_ARG(int, 18), \
         UB_ARG(int, 19), stream);                                                             \
  }
UB_MMD_THUNK(matmul_bf16)
UB_MMD_THUNK(matmul_f16)
#undef UB_MMD_THUNK

// ------------------------------------------------ GEMM launch parameters
// get_gemm_launch_params (src/gcu_device.rs:185-198) -> AtenGemmTuner::tuner
// (src/gemm_tuner.rs:326-359), which caches one GEMM_OP_PARAS
// (gemm_tuner.rs:222-258) per "type, batch, m, k, n" pattern.  Same struct
// layout and caching; the values describe this library's MI355X launch:
// sip_m x sip_n = the output tile of one workgroup, sip_k = its K-step,
// lhs/rhs/batch_multicore = the dimension with the most tiles (the grid's
// widest axis), *_pingpong = 1 (LDS ring of two or more stages).
namespace {
static_assert(sizeof(UbridgeGemmOpParas) == 132 && offsetof(UbridgeGemmOpParas, sip_m) == 32 &&
                  offsetof(UbridgeGemmOpParas, alpha) == 88 &&
                  offsetof(UbridgeGemmOpParas, input_n) == 128,
              "GEMM_OP_PARAS layout (gemm_tuner.rs:222-258)");
enum RefDataType { kDataI8 = 0, kDataFp16 = 4, kDataBf16 = 5, kDataFp32 = 8, kDataI4 = 15 };
std::mutex g_params_mu;
std::map<std::string, std::unique_ptr<UbridgeGemmOpParas>> g_params;
}  // namespace

UB_API const UbridgeGemmOpParas* ubridge_get_gemm_launch_params(int datatype, int weight_type,
                                                                size_t b, size_t m, size_t k,
                                                                size_t n, int rhs_trans) {
  const char* nm = "ubridge_get_gemm_launch_params";
  if (datatype != kDataFp16 && datatype != kDataBf16) {
    ub_set_error(UB_ERR_UNSUPPORTED, "%s: datatype %d (DataFp16 = 4, DataBf16 = 5)", nm, datatype);
    return nullptr;
  }
  if (weight_type != datatype && weight_type != kDataI8 && weight_type != kDataI4) {
    ub_set_error(UB_ERR_UNSUPPORTED, "%s: weight type %d", nm, weight_type);
    return nullptr;
  }
  if (b < 1 || m > 0x7fffffff || k > 0x7fffffff || n > 0x7fffffff || b > 0x7fffffff) {
    ub_set_error(UB_ERR_INVALID_ARG, "%s: shape b=%zu m=%zu k=%zu n=%zu", nm, b, m, k, n);
    return nullptr;
  }
  char key[128];
  snprintf(key, sizeof key, "t%d_w%d_b%zu_m%zu_k%zu_n%zu_r%d", datatype, weight_type, b, m, k, n,
           rhs_trans > 0);
  std::lock_guard<std::mutex> lk(g_params_mu);
  auto it = g_params.find(key);
  if (it != g_params.end()) return it->second.get();
  auto p = std::make_unique<UbridgeGemmOpParas>();
  memset(p.get(), 0, sizeof *p);
  int tm, tn, tk = BK;
  if (weight_type != datatype && k % 64 == 0 && n % 8 == 0 && m * b < 0x40000000ull &&
      k * n < 0x80000000ull && ub_tune(UB_TUNE_W4A16_PATH) != 1) {
    // quantized weights take the pipelined kernel of w4a16.hip (batches
    // fold into M): 256 x 256 tiles, or 128 x 256 with K split in two (64 x
    // 256 up to 64 rows).  Up to 16 rows the decode GEMV and beyond 1024 the
    // slab + hipBLASLt route run instead; the fields then name the tile the
    // pipelined kernel would use.
    tm = ub_wq_split((int)(m * b), (int)n, (int)k) ? (m * b <= 64 ? 64 : 128) : 256;
    tn = 256;
    tk = 64;
  } else {
    const int t = plan_tile((long)m, (long)n, (long)b);
    tm = t == 3 ? 256 : 128;
    tn = t == 1 ? 128 : 256;
  }
  const long mt = ub_cdiv((long)m, tm), nt = ub_cdiv((long)n, tn);
  p->input_dtype = datatype;
  p->output_dtype = datatype;
  p->csb_batch = 1;
  p->sip_batch = 1;
  p->sip_m = tm;
  p->sip_k = tk;
  p->sip_n = tn;
  p->batch_multicore = (long)b >= mt && (long)b >= nt;
  p->lhs_multicore = !p->batch_multicore && mt >= nt;
  p->rhs_multicore = !p->batch_multicore && !p->lhs_multicore;
  p->lhs_pingpong = 1;
  p->rhs_pingpong = 1;
  p->lhs_transpose = 0;
  p->rhs_transpose = rhs_trans > 0;
  p->alpha = 1.0f;
  p->input_batch = (int)b;
  p->input_m = (int)m;
  p->input_k = (int)k;
  p->input_n = (int)n;
  const UbridgeGemmOpParas* out = p.get();
  g_params.emplace(key, std::move(p));
  return out;
}
