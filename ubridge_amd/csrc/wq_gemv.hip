// wq_gemv.hip -- decode-shape (M <= 16 tokens) GEMV for the k-major
// quantized weight layouts of the W4A16 / W8A16 matmuls, gfx950.
//
//   C[M, N] = A[M, K] . deq(W)[K, N],  A / C bf16 or f16, f32 accumulate
//
// Formats (the W_* numbering of gemm.hip; scales T [K/g, N] in all):
//   0 GPTQ  int32 [K/8, N], zero points int32 [K/g, N/8]:  T((q - z) s)
//   1 U4    uint8 [K/2, N] (low nibble = even k), zeros T [K/g, N]:
//           T((q - z) s), q - z rounded in f32 first (matmul_*_4bit)
//   2 I8KN  int8 [K, N];  3 I8NK  int8 [N, K]:  T(q s)      (matmul_*_8bit)
// Scale and zero point are applied once per group to the f32 MFMA sums (see
// below), so the weight enters unrounded: outputs match the oracle to the
// GEMM tolerance, not bit for bit.
//
// Design.  With at most 16 tokens the problem is a stream of the weight
// (HBM-bound), so the kernel is shaped for bytes in flight, not for MFMA
// reuse: a workgroup owns 64 output columns and W wavefronts split K
// between them (each a contiguous range of 32-k steps, so a scale group
// stays in one wavefront); the partial sums meet in LDS in a fixed order at
// the end.  Narrow matrices also split K over workgroups (partials in a
// stream workspace, summed in split order by a second launch).  Each 32-k step of a wavefront is one
// v_mfma_f32_16x16x32 per 16-column tile with the tokens as the A rows
// (rows >= M read as zero): lane l supplies token l % 16 and the weight
// column 4 (l % 16) + j of tile j, k = 8 (l / 16) .. +7, so a lane's four
// columns are adjacent -- one 16-byte load of a GPTQ word-row, 4-byte loads
// of the byte-row layouts (16 lanes x 4 bytes = 64-byte runs per row; the
// one-shot form below stages them with swizzled 16-byte loads instead), and
// one 8-byte store per output row.  int8 [N, K] rows are read 16 k at a time
// (64-byte runs per row over the 4 lane groups); the lane's k of the two
// steps of a pair are then 16 (l / 16) + 8 s + 0..7, and its A fragments
// are loaded with the same permutation.  Two forms: k_wq_gemv holds the
// weight words of U-step batches in VGPRs, double-buffered; k_wq_gemv_os
// (the byte-row layouts, and GPTQ grids of one workgroup round) loads a
// chunk of 8 steps straight into LDS and computes each step as its loads
// land.
#include "common.h"
#include "lds_dma.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned char u8x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

enum { kGptq = 0, kU4 = 1, kI8Kn = 2, kI8Nk = 3, kDenseKn = 4, kDenseNk = 5 };
constexpr bool is_dense(int wf) { return wf == kDenseKn || wf == kDenseNk; }
constexpr uint32_t kOOB = 0x80000000u;
constexpr int kCols = 64;  // output columns per workgroup

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint64_t bytes) {
  const uint32_t n = bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)n, 0x00020000);
}
__device__ __forceinline__ uint4 ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
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
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  const f32x2 v = {lo, hi};
  if constexpr (DT == UB_BF16) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  } else {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
  }
}
template <int DT>
__device__ __forceinline__ f32x4 mfma16(const uint4& a, const uint4& b, const f32x4& c) {
  if constexpr (DT == UB_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ uint32_t half16(const uint2& v, int j) {
  const uint32_t w = j < 2 ? v.x : v.y;
  return (j & 1) ? (w >> 16) : (w & 0xffff);
}

struct WqArgs {
  const void* a;
  const void* w;
  const void* scales;
  const void* zeros;
  void* c;
  int M, N, K, group;
  float* part;  // K split over gridDim.y workgroups: f32 partials [split][M][N], else null
  int kspan;    // steps per split
  int align;    // one-shot form: wavefront step ranges start at multiples of this
};

// Raw weight words of one 32-k step for the lane's 4 columns.
//  GPTQ: 4 words (one per column, 8 k each); U4: 4 byte-rows (4 columns
//  each); I8KN: 8 byte-rows; I8NK: 2 words per column.
template <int WF>
struct Raw {
  static constexpr int NW = WF == kGptq || WF == kU4 ? 4 : is_dense(WF) ? 16 : 8;
  uint32_t w[NW];
};

// Scale epilogue per group.  The MFMA sees the weight as o + q (o = 128 for
// bf16, 1024 for f16: exact small integers built by bit operations, about
// one VALU op per value) and the f32 product P = A (o + q) is rescaled once
// per group and column: acc += s (P - (o + z) S), S = the group's sum of the
// activation row, itself an MFMA against a ones operand.  So the weight is
// used unrounded ((q - z) s exactly) where the GEMM rounds each dequantized
// value to T first; outputs agree to the GEMM tolerance, not bit for bit.
//  4-bit formats: a lane's 8 k are fed as the pairs (k, k + 4), k = 0..3, in
//  both operands: for GPTQ the pair is (w >> 4k) & 0x000f000f, for the
//  byte-row layout one v_perm joins the byte of rows p and p + 2.
//  int8: q + 128 (the sign bit flipped) converted and packed in k order.
template <int DT>
__device__ __forceinline__ uint32_t magic2() { return DT == UB_BF16 ? 0x43004300u : 0x64006400u; }
template <int DT>
__device__ __forceinline__ float magic_off() { return DT == UB_BF16 ? 128.0f : 1024.0f; }

// B operands (o + q) of a lane's 4 columns from the raw words of one step
// (m_lo = 0x000f000f, m_sg = 0x80808080, kept in VGPRs by the caller).
template <int WF, int DT>
__device__ __forceinline__ void build_b_ops(const Raw<WF>& r, uint4* b, uint32_t m_lo,
                                            uint32_t m_sg) {
  const uint32_t M2 = magic2<DT>();
  if constexpr (WF == kGptq) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t w = r.w[j];
      b[j] = make_uint4((w & m_lo) | M2, ((w >> 4) & m_lo) | M2, ((w >> 8) & m_lo) | M2,
                        ((w >> 12) & m_lo) | M2);
    }
  } else if constexpr (WF == kU4) {
    // word p = byte-row p (k 2p low nibble, 2p + 1 high); pairs (k, k + 4)
    // = rows (0, 2) and (1, 3): low nibbles, then high nibbles
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + j) << 16) | (uint32_t)j;
      const uint32_t t02 = __builtin_amdgcn_perm(r.w[2], r.w[0], sel);
      const uint32_t t13 = __builtin_amdgcn_perm(r.w[3], r.w[1], sel);
      b[j] = make_uint4((t02 & m_lo) | M2, ((t02 >> 4) & m_lo) | M2, (t13 & m_lo) | M2,
                        ((t13 >> 4) & m_lo) | M2);
    }
  } else if constexpr (WF == kDenseNk) {  // column j's 8 k are words 4j .. 4j + 3
#pragma unroll
    for (int j = 0; j < 4; j++) b[j] = make_uint4(r.w[4 * j], r.w[4 * j + 1], r.w[4 * j + 2], r.w[4 * j + 3]);
  } else if constexpr (WF == kDenseKn) {  // row q (k) holds columns 0..3 in words 2q, 2q + 1
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t sel = j & 1 ? 0x07060302u : 0x05040100u;  // high / low halves of the two rows
      uint32_t o[4];
#pragma unroll
      for (int p = 0; p < 4; p++)
        o[p] = __builtin_amdgcn_perm(r.w[2 * (2 * p + 1) + (j >> 1)], r.w[2 * (2 * p) + (j >> 1)], sel);
      b[j] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  } else {
    u8x4 X[8];
#pragma unroll
    for (int q = 0; q < 8; q++) X[q] = __builtin_bit_cast(u8x4, r.w[q] ^ m_sg);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; e++)
        v[e] = WF == kI8Kn ? (float)X[e][j] : (float)X[2 * j + (e >> 2)][e & 3];
      b[j] = make_uint4(pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]), pack2<DT>(v[4], v[5]),
                        pack2<DT>(v[6], v[7]));
    }
  }
}

// W wavefronts per workgroup, U steps per load batch.
template <int WF, int DT, int W, int U>
__global__ void __launch_bounds__(64 * W) k_wq_gemv(WqArgs p) {
  static_assert(WF != kI8Nk || U % 2 == 0, "int8 [N, K] loads cover step pairs");
  __shared__ f32x4 red[W > 1 ? W - 1 : 1][4][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, kq = lane >> 4;
  const int M = p.M, N = p.N, K = p.K;
  const int n = blockIdx.x * kCols + 4 * l16;  // the lane's first column
  const bool col_ok = n < N;                  // N % 4 == 0: all four or none
  const int nsteps = K / 32;
  const uint64_t wbytes = WF == kGptq ? (uint64_t)(K / 8) * N * 4
                          : WF == kU4 ? (uint64_t)(K / 2) * N
                          : is_dense(WF) ? (uint64_t)K * N * 2
                                         : (uint64_t)K * N;
  const __amdgpu_buffer_rsrc_t rw = rsrc(p.w, wbytes);
  const __amdgpu_buffer_rsrc_t ra = rsrc(p.a, (uint64_t)M * K * 2);
  const int ng = K / p.group;
  const __amdgpu_buffer_rsrc_t rs = rsrc(p.scales, (uint64_t)ng * N * 2);
  const __amdgpu_buffer_rsrc_t rz =
      rsrc(p.zeros, WF == kGptq ? (uint64_t)ng * (N / 8) * 4 : WF == kU4 ? (uint64_t)ng * N * 2 : 0);
  const bool row_ok = l16 < M;  // A row of this lane (token l16)
  constexpr bool kNib = WF == kGptq || WF == kU4;
  constexpr int SPU = WF == kI8Nk ? 2 : 1;  // steps per load unit (int8 [N, K]: pairs)

  // the workgroup's steps (its K split), then a contiguous range per
  // wavefront, so a scale group's steps stay together
  const int s0 = blockIdx.y * p.kspan, s1 = min(nsteps, s0 + p.kspan);
  const int per = ((s1 - s0) / SPU + W - 1) / W * SPU;
  const int t0 = s0 + wave * per, t1 = min(s1, t0 + per);

  auto load_w = [&](int t, Raw<WF>& r) {  // (int8 [N, K]: load_batch loads step pairs)
    const int k0 = 32 * t;
    if constexpr (WF == kGptq) {
      const uint4 v = ld16(rw, col_ok ? (uint32_t)(((size_t)(k0 / 8 + kq) * N + n) * 4) : kOOB);
      r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
    } else if constexpr (WF == kU4) {
#pragma unroll
      for (int q = 0; q < 4; q++)
        r.w[q] = ld4(rw, col_ok ? (uint32_t)((size_t)(k0 / 2 + 4 * kq + q) * N + n) : kOOB);
    } else if constexpr (WF == kI8Kn) {
#pragma unroll
      for (int q = 0; q < 8; q++)
        r.w[q] = ld4(rw, col_ok ? (uint32_t)((size_t)(k0 + 8 * kq + q) * N + n) : kOOB);
    } else if constexpr (WF == kDenseNk) {  // column n + j, k = k0 + 8 kq .. +7: 16 bytes
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint4 v = ld16(rw, col_ok ? (uint32_t)(((size_t)(n + j) * K + k0 + 8 * kq) * 2) : kOOB);
        r.w[4 * j] = v.x; r.w[4 * j + 1] = v.y; r.w[4 * j + 2] = v.z; r.w[4 * j + 3] = v.w;
      }
    } else if constexpr (WF == kDenseKn) {  // row k0 + 8 kq + q, columns n .. n + 3: 8 bytes
#pragma unroll
      for (int q = 0; q < 8; q++) {
        const uint2 v = ld8(rw, col_ok ? (uint32_t)(((size_t)(k0 + 8 * kq + q) * N + n) * 2) : kOOB);
        r.w[2 * q] = v.x; r.w[2 * q + 1] = v.y;
      }
    }
  };
  // A fragment of step t: token l16, k = 8 kq .. +7 (I8NK: the pair layout),
  // for the 4-bit formats reordered into the pairs (k, k + 4)
  auto load_a = [&](int t) -> uint4 {
    int k;
    if constexpr (WF == kI8Nk) k = 64 * (t >> 1) + 16 * kq + 8 * (t & 1);
    else k = 32 * t + 8 * kq;
    const uint4 x = ld16(ra, row_ok ? (uint32_t)(((size_t)l16 * K + k) * 2) : kOOB);
    if constexpr (!kNib) return x;
    return make_uint4(__builtin_amdgcn_perm(x.z, x.x, 0x05040100u),
                      __builtin_amdgcn_perm(x.z, x.x, 0x07060302u),
                      __builtin_amdgcn_perm(x.w, x.y, 0x05040100u),
                      __builtin_amdgcn_perm(x.w, x.y, 0x07060302u));
  };
  // B operands (o + q) of the lane's 4 columns
  uint32_t m_lo = 0x000f000fu, m_sg = 0x80808080u;
  asm volatile("" : "+v"(m_lo), "+v"(m_sg));
  auto build_b = [&](const Raw<WF>& r, uint4* b) { build_b_ops<WF, DT>(r, b, m_lo, m_sg); };
  // scale s and offset (o + z) of the lane's columns for group g
  auto load_sz = [&](int g, float* sc, float* oz) {
    const uint2 s = ld8(rs, col_ok ? (uint32_t)(((size_t)g * N + n) * 2) : kOOB);
#pragma unroll
    for (int j = 0; j < 4; j++) sc[j] = tof<DT>(half16(s, j));
    if constexpr (WF == kGptq) {
      const uint32_t zw = ld4(rz, col_ok ? (uint32_t)(((size_t)g * (N / 8) + n / 8) * 4) : kOOB) >>
                          (4 * (n & 7));
#pragma unroll
      for (int j = 0; j < 4; j++) oz[j] = magic_off<DT>() + (float)((zw >> (4 * j)) & 15);
    } else if constexpr (WF == kU4) {
      const uint2 z = ld8(rz, col_ok ? (uint32_t)(((size_t)g * N + n) * 2) : kOOB);
#pragma unroll
      for (int j = 0; j < 4; j++) oz[j] = (kNib ? magic_off<DT>() : 0.f) + tof<DT>(half16(z, j));
    } else {
#pragma unroll
      for (int j = 0; j < 4; j++) oz[j] = 128.0f;
    }
  };
  const uint4 ones = DT == UB_BF16 ? make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u)
                                   : make_uint4(0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u);
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc[4], P[4], S = z4;
#pragma unroll
  for (int j = 0; j < 4; j++) acc[j] = P[j] = z4;
  int cur_g = -1;
  float sc[4], oz[4];
  auto flush = [&]() {  // acc += s (P - (o + z) S); P, S cleared
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
      for (int i = 0; i < 4; i++) acc[j][i] = __builtin_fmaf(sc[j], __builtin_fmaf(-oz[j], S[i], P[j][i]), acc[j][i]);
      P[j] = z4;
    }
    S = z4;
  };

  // batches of U steps, double-buffered: the loads of the next batch are in
  // flight while this one is computed
  auto load_batch = [&](int tb, Raw<WF>* raw, uint4* af) {
#pragma unroll
    for (int i = 0; i < U; i += SPU) {
      const int t = tb + i;
      if (t < t1) {
        if constexpr (WF == kI8Nk) {  // one 16-byte load per column covers the pair
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const uint4 v = ld16(rw, col_ok ? (uint32_t)((size_t)(n + j) * K + 32 * t + 16 * kq) : kOOB);
            raw[i].w[2 * j] = v.x; raw[i].w[2 * j + 1] = v.y;
            raw[i + 1].w[2 * j] = v.z; raw[i + 1].w[2 * j + 1] = v.w;
          }
        } else {
          load_w(t, raw[i]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < U; i++)
      if (tb + i < t1) af[i] = load_a(tb + i);
  };
  auto compute_batch = [&](int tb, const Raw<WF>* raw, const uint4* af) {
#pragma unroll
    for (int i = 0; i < U; i++) {
      const int t = tb + i;
      if (t < t1) {
        uint4 b[4];
        build_b(raw[i], b);
        if constexpr (is_dense(WF)) {  // no scales: straight into the sums
#pragma unroll
          for (int j = 0; j < 4; j++) acc[j] = mfma16<DT>(af[i], b[j], acc[j]);
        } else {
          const int g = 32 * t / p.group;
          if (g != cur_g) {
            if (cur_g >= 0) flush();
            load_sz(g, sc, oz);
            cur_g = g;
          }
#pragma unroll
          for (int j = 0; j < 4; j++) P[j] = mfma16<DT>(af[i], b[j], P[j]);
          S = mfma16<DT>(af[i], ones, S);
        }
      }
    }
  };
  Raw<WF> rawA[U], rawB[U];
  uint4 afA[U], afB[U];
  if (t0 < t1) load_batch(t0, rawA, afA);
  for (int tb = t0; tb < t1; tb += 2 * U) {
    if (tb + U < t1) load_batch(tb + U, rawB, afB);
    compute_batch(tb, rawA, afA);
    if (tb + U >= t1) break;
    if (tb + 2 * U < t1) load_batch(tb + 2 * U, rawA, afA);
    compute_batch(tb + U, rawB, afB);
  }
  if (!is_dense(WF) && cur_g >= 0) flush();

  // partial sums of the W wavefronts meet in LDS, added in wave order
  if constexpr (W > 1) {
    if (wave > 0) {
#pragma unroll
      for (int j = 0; j < 4; j++) red[wave - 1][j][lane] = acc[j];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int v = 0; v < W - 1; v++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[j] += red[v][j][lane];
  }
  // lane: column l16 of each tile (n + j), tokens 4 kq + i
  if (!col_ok) return;
  if (p.part) {  // partial sums of this K split, f32
    float* P0 = p.part + (size_t)blockIdx.y * M * N;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int m = 4 * kq + i;
      if (m < M)
        *(float4*)(P0 + (size_t)m * N + n) = make_float4(acc[0][i], acc[1][i], acc[2][i], acc[3][i]);
    }
    return;
  }
  uint16_t* C = (uint16_t*)p.c;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int m = 4 * kq + i;
    if (m < M)
      *(uint2*)(C + (size_t)m * N + n) = make_uint2(pack2<DT>(acc[0][i], acc[1][i]),
                                                    pack2<DT>(acc[2][i], acc[3][i]));
  }
}

// One-shot form: every load of a wavefront's chunk of D steps is in flight
// at once.  The weight words, the chunk's activation rows and its groups'
// scales / zero points go to the wavefront's own LDS region by direct-to-LDS
// loads (no VGPRs held while they fly, and none of them a compiler-visible
// load the compiler would wait for), then one wait and the chunk's MFMAs from
// LDS.  Regions, per wavefront (bytes):
//   weights  D x SB  (SB = 1 KB per step for 4-bit, 2 KB for int8); lane i's
//            16 (or 4) bytes of instruction q at q * 1 KB (256 B) + 16 i (4 i)
//   A        ceil(M / 2) row pairs (1024 B, padded to 1040 when there are
//            several, against bank conflicts): lanes 0-31 row 2r, 32-63 row
//            2r + 1, 8 k each (512 B per row = a chunk's 256 k)
//   sz       per group of the chunk 512 B: scales (64 columns x 2 B) at +0,
//            zero points at +256 (wavefront ranges start on group
//            boundaries where a group fits a chunk, so no chunk holds a
//            partial group at each end)
// The cross-wavefront sum reuses the regions after a barrier.
template <int WF>
constexpr int os_depth() { return WF == kI8Kn ? 4 : 8; }  // steps per chunk (int8 [K, N]: 8 measured slower, fewer wavefronts fit)
template <int WF>
constexpr int os_step_bytes() { return WF == kGptq || WF == kU4 ? 1024 : 2048; }

template <int WF, int DT, int W, int D>
__global__ void __launch_bounds__(64 * W) k_wq_gemv_os(WqArgs p, int wave_bytes, int a_pairs, int pair_bytes) {
  static_assert(D % 2 == 0 && D <= 8, "a chunk's A row is one 512-byte DMA run");
  // weight load instructions per step; a chunk's loads stay within the
  // 63 that vmcnt counts
  constexpr int CPS = WF == kGptq || WF == kU4 ? 1 : 2;
  static_assert(D * CPS + 8 + 2 * (D + 1) <= 63, "vmcnt range");  // weights, A pairs, sz
  extern __shared__ __align__(16) unsigned char lds[];
  constexpr int SB = os_step_bytes<WF>();
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, kq = lane >> 4;
  const int M = p.M, N = p.N, K = p.K, group = p.group;
  // column block: consecutive blocks on one XCD (workgroup i runs on XCD
  // i % 8), so the two halves of a 128-byte line of the byte-row layouts
  // (64 columns of one byte-row) are fetched into one L2
  int cb = blockIdx.x;
  const int G8 = gridDim.x & ~7;
  if (cb < G8) cb = (cb & 7) * (G8 >> 3) + (cb >> 3);
  const int n0 = cb * kCols, n = n0 + 4 * l16;
  const bool col_ok = n < N;
  const int nsteps = K / 32, ng = K / group;
  const uint64_t wbytes = WF == kGptq ? (uint64_t)(K / 8) * N * 4
                          : WF == kU4 ? (uint64_t)(K / 2) * N
                                      : (uint64_t)K * N;
  const ub_u32x4 rw = ub_desc(p.w, wbytes);
  const ub_u32x4 ra = ub_desc(p.a, (uint64_t)M * K * 2);
  const ub_u32x4 rs = ub_desc(p.scales, (uint64_t)ng * N * 2);
  const ub_u32x4 rz = ub_desc(p.zeros, WF == kGptq ? (uint64_t)ng * (N / 8) * 4
                                       : WF == kU4 ? (uint64_t)ng * N * 2 : 0);
  constexpr bool kNib = WF == kGptq || WF == kU4;
  constexpr int SPU = WF == kI8Nk ? 2 : 1;
  const uint32_t base = ub_lds_addr(lds) + (uint32_t)(wave * wave_bytes);
  const uint32_t wreg = base, areg = base + D * SB, szreg = areg + a_pairs * pair_bytes;

  const int s0 = blockIdx.y * p.kspan, s1 = min(nsteps, s0 + p.kspan);
  const int per = ((s1 - s0) / p.align + W - 1) / W * p.align;
  const int t0 = s0 + wave * per, t1 = min(s1, t0 + per);

  // per-lane DMA offsets at step 0 (the step's offset is the scalar part)
  uint32_t vw[8];
  if constexpr (WF == kGptq) vw[0] = col_ok ? (uint32_t)(((size_t)kq * N + n) * 4) : kOOB;
#pragma unroll
  for (int q = 0; q < 8; q++) {
    if constexpr (WF == kU4) {
      // one 16-byte load per lane and step: lane L fetches byte-row 4 ((L / 4) % 4) +
      // L / 16, columns 16 (L % 4) .. +15, so LDS unit L holds (row r, chunk c) at
      // 16 (r % 4) + 4 (r / 4) + c and the 64 lanes reading one of their byte-rows
      // hit 64 different banks
      if (q == 0) {
        const int row = 4 * ((lane >> 2) & 3) + (lane >> 4), ch = lane & 3;
        vw[0] = n0 + 16 * ch < N ? (uint32_t)((size_t)row * N + n0 + 16 * ch) : kOOB;
      }
    }
    if constexpr (WF == kI8Kn) {
      // two 16-byte loads per lane and step: unit u = 64 q + lane (q < 2)
      // holds row 8 ((u / 4) % 4) + u / 16, columns 16 (u % 4) .. +15, i.e.
      // (row r, chunk c) at 16 (r % 8) + 4 (r / 8) + c: bank-conflict-free
      // reads of one byte-row by the 64 lanes
      if (q < 2) {
        const int u = 64 * q + lane, row = 8 * ((u >> 2) & 3) + (u >> 4), ch = u & 3;
        vw[q] = n0 + 16 * ch < N ? (uint32_t)((size_t)row * N + n0 + 16 * ch) : kOOB;
      }
    }
    if constexpr (WF == kI8Nk) { if (q < 4) vw[q] = col_ok ? (uint32_t)((size_t)(n + q) * K + 16 * kq) : kOOB; }
  }
  const int arow = lane >> 5, ak = 8 * (lane & 31);  // A DMA: row 2r + arow, k ak .. +7
  const bool s_ok = lane < 32 && n0 + 2 * lane < N;
  const bool z_ok = WF == kGptq ? lane < 8 && n0 / 8 + lane < N / 8
                                : WF == kU4 && lane < 32 && n0 + 2 * lane < N;

  const uint4 ones = DT == UB_BF16 ? make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u)
                                   : make_uint4(0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u);
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc[4], P[4], S = z4;
#pragma unroll
  for (int j = 0; j < 4; j++) acc[j] = P[j] = z4;
  float sc[4], oz[4];
  uint32_t m_lo = 0x000f000fu, m_sg = 0x80808080u;
  asm volatile("" : "+v"(m_lo), "+v"(m_sg));
  auto flush = [&]() {
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
      for (int i = 0; i < 4; i++)
        acc[j][i] = __builtin_fmaf(sc[j], __builtin_fmaf(-oz[j], S[i], P[j][i]), acc[j][i]);
      P[j] = z4;
    }
    S = z4;
  };

  for (int c0 = t0; c0 < t1; c0 += D) {
    const int c1 = min(t1, c0 + D);
    const int g0 = 32 * c0 / group, g1 = (32 * c1 - 1) / group;
    // ---- issue: activations, scales / zeros, then the weights
    for (int r = 0; r < a_pairs; r++) {
      const int row = 2 * r + arow, k = 32 * c0 + ak;
      ub_lds_load16_at(ra, areg + r * pair_bytes,
                       row < M && k < 32 * c1 ? (uint32_t)(((size_t)row * K + k) * 2) : kOOB, 0);
    }
    for (int g = g0; g <= g1; g++) {
      const uint32_t dst = szreg + (g - g0) * 512;
      ub_lds_load4_at(rs, dst, s_ok ? (uint32_t)(((size_t)g * N + n0) * 2 + 4 * lane) : kOOB, 0);
      if constexpr (WF == kGptq)
        ub_lds_load4_at(rz, dst + 256,
                        z_ok ? (uint32_t)(((size_t)g * (N / 8) + n0 / 8 + lane) * 4) : kOOB, 0);
      if constexpr (WF == kU4)
        ub_lds_load4_at(rz, dst + 256, z_ok ? (uint32_t)(((size_t)g * N + n0) * 2 + 4 * lane) : kOOB,
                        0);
    }
    for (int t = c0; t < c1; t += SPU) {
      const uint32_t dst = wreg + (t - c0) * SB;
      if constexpr (WF == kGptq) {
        ub_lds_load16_at(rw, dst, vw[0], (uint32_t)(16 * t) * (uint32_t)N);
      } else if constexpr (WF == kU4) {
        ub_lds_load16_at(rw, dst, vw[0], (uint32_t)(16 * t) * (uint32_t)N);
      } else if constexpr (WF == kI8Kn) {
#pragma unroll
        for (int q = 0; q < 2; q++) ub_lds_load16_at(rw, dst + q * 1024, vw[q], (uint32_t)(32 * t) * (uint32_t)N);
      } else {
#pragma unroll
        for (int j = 0; j < 4; j++) ub_lds_load16_at(rw, dst + j * 1024, vw[j], (uint32_t)(32 * t));
      }
    }
    // ---- compute from LDS, step i once its loads have landed (loads
    // complete in issue order: activations and scales first, then the
    // weights step by step, CPS instructions each)
    int cur_g = -1, next_t = c0;  // next_t: the first step of the next group
    auto step = [&](int t) {
      if (t == next_t) {
        const int g = 32 * t / group;
        next_t = (g + 1) * (group / 32);
        if (cur_g >= 0) flush();
        const uint32_t sz = szreg + (g - g0) * 512;
        const uint2 sv = ub_lds_read8(sz + 8 * l16);
#pragma unroll
        for (int j = 0; j < 4; j++) sc[j] = tof<DT>(half16(sv, j));
        if constexpr (WF == kGptq) {
          const uint32_t zw = ub_lds_read4(sz + 256 + 4 * (l16 >> 1)) >> (16 * (l16 & 1));
#pragma unroll
          for (int j = 0; j < 4; j++) oz[j] = magic_off<DT>() + (float)((zw >> (4 * j)) & 15);
        } else if constexpr (WF == kU4) {
          const uint2 zv = ub_lds_read8(sz + 256 + 8 * l16);
#pragma unroll
          for (int j = 0; j < 4; j++) oz[j] = magic_off<DT>() + tof<DT>(half16(zv, j));
        } else {
#pragma unroll
          for (int j = 0; j < 4; j++) oz[j] = 128.0f;
        }
        cur_g = g;
      }
      Raw<WF> r;
      const uint32_t src = wreg + (t - c0) * SB;
      if constexpr (WF == kGptq) {
        const uint4 v = ub_lds_read16(src + 16 * lane);
        r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
      } else if constexpr (WF == kU4) {  // byte-row 4 kq + q: unit 16 q + 4 kq + l16 / 4
#pragma unroll
        for (int q = 0; q < 4; q++)
          r.w[q] = ub_lds_read4(src + (16 * q + 4 * kq + (l16 >> 2)) * 16 + 4 * (l16 & 3));
      } else if constexpr (WF == kI8Kn) {  // byte-row 8 kq + q: unit 16 q + 4 kq + l16 / 4
#pragma unroll
        for (int q = 0; q < 8; q++)
          r.w[q] = ub_lds_read4(src + (16 * q + 4 * kq + (l16 >> 2)) * 16 + 4 * (l16 & 3));
      } else {
        const uint32_t pb = wreg + ((t - c0) & ~1) * SB + 16 * lane + 8 * (t & 1);
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const uint2 v = ub_lds_read8(pb + j * 1024);
          r.w[2 * j] = v.x; r.w[2 * j + 1] = v.y;
        }
      }
      // A fragment: token l16, k = 8 kq .. +7 of the step (int8 [N, K]: the
      // pair layout), 4-bit formats reordered into the pairs (k, k + 4)
      int kl;
      if constexpr (WF == kI8Nk) kl = 64 * ((t - c0) >> 1) + 16 * kq + 8 * (t & 1);
      else kl = 32 * (t - c0) + 8 * kq;
      uint4 x = make_uint4(0, 0, 0, 0);
      if (l16 < M) x = ub_lds_read16(areg + (l16 >> 1) * pair_bytes + (l16 & 1) * 512 + 2 * kl);
      uint4 af = x;
      if constexpr (kNib)
        af = make_uint4(__builtin_amdgcn_perm(x.z, x.x, 0x05040100u),
                        __builtin_amdgcn_perm(x.z, x.x, 0x07060302u),
                        __builtin_amdgcn_perm(x.w, x.y, 0x05040100u),
                        __builtin_amdgcn_perm(x.w, x.y, 0x07060302u));
      uint4 b[4];
      build_b_ops<WF, DT>(r, b, m_lo, m_sg);
#pragma unroll
      for (int j = 0; j < 4; j++) P[j] = mfma16<DT>(af, b[j], P[j]);
      S = mfma16<DT>(af, ones, S);
    };
    // a full chunk waits step by step (vmcnt takes an immediate: one wait
    // per step index), a short one for all its loads at once
    const bool full = c1 - c0 == D;
#pragma unroll 1
    for (int i = 0; i < c1 - c0; i++) {
      const int left = !full ? 0 : WF == kI8Nk ? (D / 2 - 1 - i / 2) * 4 : (D - 1 - i) * CPS;
      switch (left) {
#define UB_OS_WAIT(n) case n: ub_wait_vmcnt<n>(); break;
        UB_OS_WAIT(1) UB_OS_WAIT(2) UB_OS_WAIT(3) UB_OS_WAIT(4) UB_OS_WAIT(5) UB_OS_WAIT(6)
        UB_OS_WAIT(7) UB_OS_WAIT(8) UB_OS_WAIT(12) UB_OS_WAIT(16) UB_OS_WAIT(20) UB_OS_WAIT(24)
        UB_OS_WAIT(28)
#undef UB_OS_WAIT
        default: ub_wait_vmcnt<0>(); break;
      }
      step(c0 + i);
    }
    if (cur_g >= 0) flush();
  }

  // partial sums of the W wavefronts meet in LDS (the regions are free once
  // every wavefront is past its last chunk); then each of the workgroup's
  // threads adds up one output, in wave order
  if constexpr (W > 1) {
    f32x4* red = (f32x4*)lds;  // [W][4][64]
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; j++) red[(wave * 4 + j) * 64 + lane] = acc[j];
    __syncthreads();
    const int Mr = min(M, 16);
    for (int o = threadIdx.x; o < Mr * kCols; o += 64 * W) {
      const int m = o / kCols, c = o % kCols, col = n0 + c;
      const int ln = c / 4 + 16 * (m / 4), j = c % 4, i = m % 4;
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < W; w++) v += red[(w * 4 + j) * 64 + ln][i];
      if (col < N) {
        if (p.part) p.part[((size_t)blockIdx.y * M + m) * N + col] = v;
        else ((uint16_t*)p.c)[(size_t)m * N + col] = (uint16_t)(pack2<DT>(v, 0.f) & 0xffff);
      }
    }
    return;
  }
  if (!col_ok) return;
  if (p.part) {
    float* P0 = p.part + (size_t)blockIdx.y * M * N;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int m = 4 * kq + i;
      if (m < M)
        *(float4*)(P0 + (size_t)m * N + n) = make_float4(acc[0][i], acc[1][i], acc[2][i], acc[3][i]);
    }
    return;
  }
  uint16_t* C = (uint16_t*)p.c;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int m = 4 * kq + i;
    if (m < M)
      *(uint2*)(C + (size_t)m * N + n) = make_uint2(pack2<DT>(acc[0][i], acc[1][i]),
                                                    pack2<DT>(acc[2][i], acc[3][i]));
  }
}

// out[m, n] = T(sum over the splits of part[split][m][n]), in split order;
// four columns per thread
template <int DT>
__global__ void __launch_bounds__(256) k_wq_reduce(const float* __restrict__ part,
                                                   uint16_t* __restrict__ out, int MN4, int splits) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= MN4) return;
  float4 v = ((const float4*)part)[i];
  for (int sp = 1; sp < splits; sp++) {
    const float4 u = ((const float4*)part)[(size_t)sp * MN4 + i];
    v.x += u.x; v.y += u.y; v.z += u.z; v.w += u.w;
  }
  ((uint2*)out)[i] = make_uint2(pack2<DT>(v.x, v.y), pack2<DT>(v.z, v.w));
}

template <int WF, int DT, int W>
void launch_os(const WqArgs& p, dim3 grid, int wave_bytes, int a_pairs, int pair_bytes,
               hipStream_t s) {
  constexpr int D = os_depth<WF>();
  const int lds = W * wave_bytes;
  (void)hipFuncSetAttribute((const void*)k_wq_gemv_os<WF, DT, W, D>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  k_wq_gemv_os<WF, DT, W, D><<<grid, 64 * W, lds, s>>>(p, wave_bytes, a_pairs, pair_bytes);
}

template <int WF, int DT>
int launch_one_shot(WqArgs p, hipStream_t s) {
  constexpr int D = os_depth<WF>();
  constexpr int SPU = WF == kI8Nk ? 2 : 1;
  const int wgs = ub_cdiv(p.N, kCols), steps = p.K / 32;
  // wavefront ranges start on a group boundary when a group is at most a
  // chunk, so a chunk holds D * 32 / group groups, not one more
  const int gs = p.group / 32;
  int al = gs <= D ? gs : 1;
  if (al % SPU) al *= SPU;
  const bool aligned = gs <= D && D % al == 0;
  const int gmax = (32 * D + p.group - 1) / p.group + (aligned ? 0 : 1);
  p.align = aligned ? al : SPU;
  const int a_pairs = (p.M + 1) / 2;
  const int pair_bytes = a_pairs > 1 ? 1040 : 1024;  // pairs padded against bank conflicts
  const int wave_bytes = D * os_step_bytes<WF>() + a_pairs * pair_bytes + gmax * 512;
  int W = 16;
  while (W > 1 && W * wave_bytes > 160 * 1024) W /= 2;
  int splits = 1;  // narrow matrices: K over up to 256 workgroups as in launch()
  while (wgs < 128 && splits < 8 && wgs * splits < 256 && steps / (2 * splits * W) >= 2)
    splits *= 2;
  p.part = nullptr;
  p.kspan = steps;
  UbScratch ws(s, splits > 1 ? (size_t)splits * p.M * p.N * sizeof(float) : 0);
  if (splits > 1) {
    p.part = (float*)ws.get();
    if (p.part) p.kspan = (steps / p.align + splits - 1) / splits * p.align;
    else splits = 1;
  }
  dim3 grid(wgs, splits);
  switch (W) {
    case 16: launch_os<WF, DT, 16>(p, grid, wave_bytes, a_pairs, pair_bytes, s); break;
    case 8: launch_os<WF, DT, 8>(p, grid, wave_bytes, a_pairs, pair_bytes, s); break;
    case 4: launch_os<WF, DT, 4>(p, grid, wave_bytes, a_pairs, pair_bytes, s); break;
    case 2: launch_os<WF, DT, 2>(p, grid, wave_bytes, a_pairs, pair_bytes, s); break;
    default: launch_os<WF, DT, 1>(p, grid, wave_bytes, a_pairs, pair_bytes, s); break;
  }
  if (splits > 1) {
    const int mn4 = p.M * p.N / 4;
    k_wq_reduce<DT><<<ub_cdiv(mn4, 256), 256, 0, s>>>(p.part, (uint16_t*)p.c, mn4, splits);
  }
  return ub_check_launch("quantized gemv");
}

template <int WF, int DT>
int launch(WqArgs p, hipStream_t s) {
  // the one-shot form for the byte-row layouts (measured on MI355X at the
  // Llama-3-8B shapes, 1-16 tokens: uint8 4-bit 16.2 -> 13.1 us, int8
  // [K, N] 23.8 -> 20.9 us at 4096 x 14336) and for GPTQ when its grid is one
  // round of workgroups (11.5 -> 10.3 us); int8 [N, K] and wider GPTQ grids
  // keep the register-batched form, measured faster there
  if constexpr (WF == kU4 || WF == kI8Kn || WF == kGptq) {
    // (the byte-row layouts: 16-byte loads of 16-column chunks, so N % 16 ==
    // 0 keeps them 16-byte aligned)
    if ((WF != kGptq || ub_cdiv(p.N, kCols) <= 256) && (WF == kGptq || p.N % 16 == 0))
      return launch_one_shot<WF, DT>(p, s);
  }
  // wavefronts per workgroup (one workgroup per 64 columns): 16 while the
  // grid has fewer workgroups than CUs, else 8 -- the byte-row layouts keep
  // 8 (more VGPRs per lane) -- and each wavefront with at least 4 steps;
  // two steps per load batch, double-buffered (measured on MI355X at the
  // Llama-3-8B shapes: deeper batches and 4-wavefront groups were slower)
  const int wgs = ub_cdiv(p.N, kCols), steps = p.K / 32;
  int W = wgs < 256 && (WF == kGptq || WF == kI8Nk) ? 16 : 8;
  while (W > 1 && steps / W < 4) W /= 2;
  // Narrow matrices (fewer than 128 column workgroups): K split over
  // workgroups up to 256 of them (each wavefront keeping >= 4 steps),
  // partials through a stream workspace and summed in split order by a second
  // launch; if that scratch cannot be allocated, the single-launch form.  (Measured: GPTQ 14336 x 4096 at one token
  // 25.5 -> 13.7 us; at N = 14336 and wider the second launch costs more than
  // the split gains.)
  constexpr int SPU = WF == kI8Nk ? 2 : 1;
  int splits = 1;
  while (wgs < 128 && splits < 8 && wgs * splits < 256 && steps / (2 * splits * W) >= 4)
    splits *= 2;
  p.part = nullptr;
  p.kspan = steps;
  UbScratch ws(s, splits > 1 ? (size_t)splits * p.M * p.N * sizeof(float) : 0);
  if (splits > 1) {
    p.part = (float*)ws.get();
    if (p.part) p.kspan = (steps / SPU + splits - 1) / splits * SPU;
    else splits = 1;
  }
  dim3 grid(wgs, splits);
  constexpr int U = 2;
  switch (W) {
    case 16: k_wq_gemv<WF, DT, 16, U><<<grid, 1024, 0, s>>>(p); break;
    case 8: k_wq_gemv<WF, DT, 8, U><<<grid, 512, 0, s>>>(p); break;
    case 4: k_wq_gemv<WF, DT, 4, U><<<grid, 256, 0, s>>>(p); break;
    case 2: k_wq_gemv<WF, DT, 2, U><<<grid, 128, 0, s>>>(p); break;
    default: k_wq_gemv<WF, DT, 1, U><<<grid, 64, 0, s>>>(p); break;
  }
  if (splits > 1) {
    const int mn4 = p.M * p.N / 4;
    k_wq_reduce<DT><<<ub_cdiv(mn4, 256), 256, 0, s>>>(p.part, (uint16_t*)p.c, mn4, splits);
  }
  return ub_check_launch("quantized gemv");
}

}  // namespace

// Decode-shape GEMV for the k-major quantized layouts (wf: 0 GPTQ, 1 uint8
// [K/2, N] 4-bit, 2 int8 [K, N], 3 int8 [N, K]); returns UB_ERR_UNSUPPORTED
// (without recording an error) outside its contract: M <= 16, K and group
// multiples of 32 (64 for wf 3), N a multiple of 4.
int ub_wq_gemv(int wf, const void* a, const void* w, const void* scales, const void* zeros,
               void* out, int M, int K, int N, int group, int dtype, hipStream_t s) {
  // int8 [N, K] steps come in pairs whose k interleave over 64: its groups
  // must hold whole pairs
  if (M < 1 || M > 16 || K % (wf == kI8Nk ? 64 : 32) != 0 || K < 32 ||
      group % (wf == kI8Nk ? 64 : 32) != 0 ||
      N % 4 != 0 || wf < 0 || wf > 5)
    return UB_ERR_UNSUPPORTED;
  if ((uint64_t)M * K * 2 >= 0x80000000ull || (uint64_t)K * N * (wf >= 4 ? 2 : 1) >= 0x80000000ull ||
      (uint64_t)(K / group) * N * 2 >= 0x80000000ull)
    return UB_ERR_UNSUPPORTED;  // 32-bit buffer offsets
  WqArgs p{a, w, scales, zeros, out, M, N, K, group, nullptr, K / 32, 1};
#define UB_WQ(F)                                                              \
  if (wf == F) return dtype == UB_BF16 ? launch<F, UB_BF16>(p, s) : launch<F, UB_F16>(p, s);
  UB_WQ(kGptq) UB_WQ(kU4) UB_WQ(kI8Kn) UB_WQ(kI8Nk) UB_WQ(kDenseKn) UB_WQ(kDenseNk)
#undef UB_WQ
  return UB_ERR_UNSUPPORTED;
}
