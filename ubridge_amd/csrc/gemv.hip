// gemv.hip -- fused dequant + decode GEMV (M <= 16 tokens) for GGUF Q4_0,
// Q8_0 and Q4_K weights in the reference SoA layout, on gfx950.
//
// Replaces Candle's QMatMul on the GCU, which the reference serves as
// "dequantize whole weight (quant.cpp:257-268, 486-488) -> dense matmul
// (matmul.cpp:1143-1184)" and so moves the weight through HBM three times.
// Here the weight is read once, straight from its packed blocks.
//
// Numerics follow Candle's CPU QMatMul (k_quants::matmul): each activation
// row is quantized to the weight's vec-dot type (Q8_0 per 32 for Q4_0/Q8_0,
// Q8_K per 256 for Q4_K), each block dot is an exact integer (v_dot4_i32_i8),
// and the per-block integer is scaled in f32 exactly as Candle's generic
// vec_dot does: (float)sumi * d_w * d_a.  Only the order in which block
// results are summed differs (lanes, then a wave butterfly).
//
// Mapping: a 256-thread workgroup holds 4 wavefronts; each wavefront owns R
// consecutive weight rows, and its 64 lanes stride along K so that every
// 16-byte load of a wavefront covers 1 KiB of contiguous codes.  The quantized
// activations (a few KiB per token) are re-read from L1/L2 once per R rows.
#include "common.h"
#include "lds_dma.h"

int ub_quantize_act_q8_0(const void* x, int x_dt, size_t n, int8_t* q, float* d, int* s,
                         hipStream_t st);
int ub_quantize_act_q8_k(const void* x, int x_dt, size_t n, int8_t* q, float* d, int* bs,
                         hipStream_t st);

// gemm.hip: GEMM on a GGUF weight dequantized into LDS tile by tile
bool ub_gguf_pipelined_fits(int qtype, int M, int N, int K);
int ub_gguf_pipelined(int qtype, const void* w, const void* x, void* y, int y_f32, int M, int N,
                      int K, bool may_alloc, hipStream_t s);
int ub_gguf_gemm(int qtype, const void* w, const void* x, void* y, int y_f32, int M, int N, int K,
                 hipStream_t s);
// quant.hip: rows of a GGUF weight dequantized (the dequantize_block_* values)
int ub_dequant_rows(int qtype, const void* w, int N, int K, int r0, int nrows, void* out, int dt,
                    hipStream_t s);
// blaslt.cpp: plain library GEMM
bool ub_blaslt_ready(int batch, int M, int N, int K, int rhs_t, int bcast, int ldc, int c_f32,
                     int dt, hipStream_t s);
int ub_blaslt_gemm(const void* a, const void* b, void* c, int batch, int M, int N, int K,
                   int rhs_t, int bcast, int ldc, int c_f32, int dt, hipStream_t s);

namespace {

constexpr int kWaves = 4;

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
// Streaming (non-temporal) 16-byte load: weights are touched once per call.
__device__ __forceinline__ uint4 ld_nt(const uint4* p) {
  u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

struct ActWs {
  int8_t* q;
  float* d;
  int* s;  // per-32-element code sums (Q8_0 blocks / Q8_K sub-blocks)
};

inline size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

ActWs carve(void* ws, int qt, int M, int K) {
  uint8_t* p = (uint8_t*)ws;
  size_t n = (size_t)M * K;
  ActWs a;
  a.q = (int8_t*)p;
  p += al256(n);
  a.d = (float*)p;
  p += al256(sizeof(float) * (qt == UB_Q4_K ? n / 256 : n / 32));
  a.s = (int*)p;
  return a;
}

size_t ws_size(int qt, int M, int K) {
  size_t n = (size_t)M * K;
  if (qt == UB_Q4_K) return al256(n) + al256(4 * (n / 256)) + al256(4 * (n / 32));
  return al256(n) + al256(4 * (n / 32)) + al256(4 * (n / 32));
}

// From qmm_lib_m(qtype) tokens on, ubridge_qmatmul computes the reference's GCU
// sequence (dequantize_block_*_bf16, then a bf16 GEMM): the weight is
// dequantized slab by slab (at most kQmmSlabBytes of bf16) into the
// per-stream library workspace and each slab multiplied by hipBLASLt, since
// the GEMV re-reads the weight once per 16 tokens.  Where that is not
// available (hipBLASLt has no algorithm for the shape, the scratch
// allocation failed, or the allocation-free entry point) it runs, from kQmmGemmM tokens on, one MFMA-core
// GEMM that dequantizes the weight tile by tile in LDS (the same values, no
// HBM copy), else the GEMV.  Measured on MI355X at 4096 x 14336 (us; GEMV /
// LDS-dequant GEMM / dequantize + hipBLASLt): Q4_K 32 tokens 29 / - / 50, 64
// 54 / - / 52, 128 106 / 124 / 54, 512 423 / 137 / 81, 2048 - / 488 / 221;
// Q8_0 32 42 / - / 50, 63 80 / - / 53, 512 619 / 137 / 82.  A slab of up to
// 256 MB keeps the common shapes to one hipBLASLt call (64 MB slabs: 2 calls
// at 4096 x 14336, 52 -> 79 us at 64 tokens).
constexpr int kQmmGemmM = 128;
// Q4_K 4096 x 14336, bf16 x (us, pipelined GEMM -- K split over workgroups
// where its grid is small -- / slab + hipBLASLt): 64 tokens 30.5 / 49.4,
// 128 38.3 / 52.8, 256 53.4 / 66.6, 512 78.9 / 81.8, 768 114.9 / 108.7,
// 1024 128 / 123
constexpr int kGgufFusedHi = 768;
// Fewest tokens for which that GEMM (K split over workgroups, 64-row tiles
// up to 64 tokens) beats the 16-token GEMV passes: 4096 x 14336 / 4096 x
// 4096, us, GEMV / pipelined: Q4_0 17 tokens 39.8 / 19.7, 25.9 / 14.1; 32
// 67.8 / 21.9, 42.5 / 15.0.  Q8_0 17 35.5 / 23.4, 15.9 / 14.5; 32 41.6 /
// 24.7, 17.9 / 15.4.  Q4_K 17 21.9 / 20.8, 11.8 / 14.5; 32 28.2 / 22.9,
// 14.3 / 15.4; 40 40.3 / 23.8, 20.1 / 15.9.
int qmm_fused_m(int qt, int N) { return qt == UB_Q4_K && N < 8192 ? 40 : 17; }
constexpr size_t kQmmSlabBytes = 256ull << 20;
int qmm_lib_m(int qt) { return qt == UB_Q4_K ? 64 : 40; }
// workspace of ubridge_qmatmul: the quantized activations, or on the GEMM
// routes the bf16 copy of f32 activations -- possible from 17 tokens, or
// from qmm_lib_m when the call may not allocate (ubridge_qmatmul_noalloc)
size_t qmm_ws_size(int qt, int M, int K, bool may_alloc = true) {
  const size_t w = ws_size(qt, M, K);
  const bool gemm = may_alloc ? M > 16 : M >= qmm_lib_m(qt);
  return gemm ? (w > al256((size_t)M * K * 2) ? w : al256((size_t)M * K * 2)) : w;
}

__global__ void __launch_bounds__(256) k_f32_to_bf16(const float* __restrict__ x,
                                                     uint16_t* __restrict__ y, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    y[i] = ub_f32_to_bf16(x[i]);
}

// bf16 / f16 elements copied one by one (x may be only 2-byte aligned)
__global__ void __launch_bounds__(256) k_b16_copy(const uint16_t* __restrict__ x,
                                                  uint16_t* __restrict__ y, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    y[i] = x[i];
}

__global__ void k_zero(uint8_t* p, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

template <int OT>
__device__ __forceinline__ void store_out(void* y, size_t i, float v) {
  if constexpr (OT == UB_F32) ((float*)y)[i] = v;
  else ((uint16_t*)y)[i] = ub_f32_to_bf16(v);
}

// ------------------------------------------------------ wave reduction
// Reduce-scatter butterfly over NV = R*MT partial sums held by every lane:
// at each of the first log2(NV) steps a lane keeps half of its values and
// receives its partner's copy of that half, so NV values cost NV-1 + (6 -
// log2 NV) exchanges instead of 6*NV.  Afterwards lane L holds the wave total
// of value index L >> (6 - log2 NV) in v[0].
//
// Exchanges are cross-lane VALU ops, not LDS permutes: the 32- and 16-lane
// steps use v_permlane32_swap / v_permlane16_swap, which swap one register's
// upper half (odd rows) with another's lower half (even rows), so a single
// swap of the pair (v[i], v[i + c/2]) hands each half the partner copy it
// needs.  The 8-, 4-, 2- and 1-lane steps use DPP row_mirror (partner
// L ^ 15), row_half_mirror (L ^ 7) and quad_perm (L ^ 2, L ^ 1): each flips
// the step's lane bit, and together they span all 16 lanes of a row.
__device__ __forceinline__ float f_of(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t u_of(float f) { return __float_as_uint(f); }

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

template <int STEP>
__device__ __forceinline__ void swap_add(float& lo, float& hi) {
  if constexpr (STEP == 0) {
    auto r = __builtin_amdgcn_permlane32_swap(u_of(lo), u_of(hi), false, false);
    lo = f_of(r[0]) + f_of(r[1]);
  } else {
    auto r = __builtin_amdgcn_permlane16_swap(u_of(lo), u_of(hi), false, false);
    lo = f_of(r[0]) + f_of(r[1]);
  }
}

template <int NV>
__device__ __forceinline__ float wave_reduce_scatter(float (&v)[NV], int lane) {
  static_assert(NV >= 1 && NV <= 64 && (NV & (NV - 1)) == 0, "NV must be a power of two <= 64");
  // lane steps 32 and 16: permlane swaps
#pragma unroll
  for (int step = 0; step < 2; step++) {
    const int c = (NV >> step) > 1 ? (NV >> step) : 1;
#pragma unroll
    for (int i = 0; i < (c > 1 ? c / 2 : 1); i++) {
      float& a = v[i];
      float b = c > 1 ? v[i + c / 2] : v[i];
      if (step == 0) swap_add<0>(a, b);
      else swap_add<1>(a, b);
    }
  }
  // lane steps 8, 4, 2, 1: DPP partners L^15, L^7, L^2, L^1
#pragma unroll
  for (int step = 2; step < 6; step++) {
    const int off = 32 >> step;
    const int c = (NV >> step) > 1 ? (NV >> step) : 1;
    const bool upper = (lane & off) != 0;
#pragma unroll
    for (int i = 0; i < (c > 1 ? c / 2 : 1); i++) {
      const float send = c > 1 ? (upper ? v[i] : v[i + c / 2]) : v[i];
      const float keep = c > 1 ? (upper ? v[i + c / 2] : v[i]) : v[i];
      float recv;
      if (step == 2) recv = dpp_f<0x140>(send);       // row_mirror
      else if (step == 3) recv = dpp_f<0x141>(send);  // row_half_mirror
      else if (step == 4) recv = dpp_f<0x4E>(send);   // quad_perm [2,3,0,1]
      else recv = dpp_f<0xB1>(send);                  // quad_perm [1,0,3,2]
      v[i] = keep + recv;
    }
  }
  return v[0];
}

template <int N>
constexpr int ilog2() { return N <= 1 ? 0 : 1 + ilog2<N / 2>(); }

// ----------------------------------------------------------- block codecs
// Q4_0 / Q8_0: one lane per 32-element block.  Q4_0: 16 code bytes (low
// nibbles of dword i = elements 4i..4i+3, high nibbles 16+4i..), and
// sum (q-8)*a = sum lo*a - 8*sum a[0..15] + sum (hi-8)*a[16..31], with the
// sum of the first 16 activation codes kept in the workspace.
// Q4_K: four lanes (a quad) per 256-element super-block; lane t = lane%4 reads
// code bytes [32t, 32t+32): their low nibbles are elements 64t+(0..31)
// (sub-block 2t), their high nibbles 64t+32+(0..31) (sub-block 2t+1).  Per
// block and token:
//   d_w*d_a*(sc_lo*dot_lo + sc_hi*dot_hi) - dmin_w*d_a*(m_lo*s_lo + m_hi*s_hi)
// with s the 32-element activation code sums.  Every dot is an exact int32.
//
// Weights are read with raw buffer loads through a descriptor covering
// exactly the wavefront's rows; a block past the end of K or a row past N
// gets offset kOOB, which reads zero without touching memory.  The loads
// therefore need no branches, and the compiler keeps them all in flight (a
// branch around a load forces a full vmcnt(0) wait at the join).
typedef unsigned int u32x4b __attribute__((ext_vector_type(4)));
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer, 32-bit data format (gfx9)
constexpr int kAuxNT = 2;               // non-temporal: weights are read once
constexpr uint32_t kOOB = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kRsrcWord3);
}
// Same, with every field forced wave-uniform (readfirstlane): for operands the
// compiler cannot prove uniform, so that it keeps the descriptor in SGPRs
// instead of wrapping each load in a waterfall loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_u(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  return rsrc((const void*)(((uint64_t)hi << 32) | lo), __builtin_amdgcn_readfirstlane(bytes));
}
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  u32x4b v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kAuxNT);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 bload8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  typedef unsigned int u32x2b __attribute__((ext_vector_type(2)));
  u32x2b v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t bload4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t bload2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}

struct WReg {
  uint4 q0, q1;  // codes (q1: second 16 bytes for Q8_0 and Q4_K)
  uint32_t h;    // Q4_0/Q8_0: fp16 scale bits; Q4_K: header dword t
};

template <int QT>
struct Geo {
  static constexpr int LPB = QT == UB_Q4_K ? 4 : 1;   // lanes per block
  static constexpr int BK = QT == UB_Q4_K ? 256 : 32;
  static constexpr int BPI = 64 / LPB;                // blocks per wave iteration
  static constexpr int QB = QT == UB_Q4_K ? 128 : (QT == UB_Q8_0 ? 32 : 16);  // code bytes
  static constexpr int HB = QT == UB_Q4_K ? 16 : 2;    // header bytes
};

template <int QT>
__device__ __forceinline__ void load_w(WReg& r, __amdgpu_buffer_rsrc_t q, __amdgpu_buffer_rsrc_t h,
                                       uint32_t b, bool ok, int t) {
  if constexpr (QT == UB_Q4_0) {
    r.q0 = bload16(q, ok ? b * 16 : kOOB);
    r.h = bload2(h, ok ? b * 2 : kOOB);
  } else if constexpr (QT == UB_Q8_0) {
    r.q0 = bload16(q, ok ? b * 32 : kOOB);
    r.q1 = bload16(q, ok ? b * 32 + 16 : kOOB);
    r.h = bload2(h, ok ? b * 2 : kOOB);
  } else {
    r.q0 = bload16(q, ok ? b * 128 + t * 32 : kOOB);
    r.q1 = bload16(q, ok ? b * 128 + t * 32 + 16 : kOOB);
    r.h = bload4(h, ok ? b * 16 + t * 4 : kOOB);
  }
}

__device__ __forceinline__ int dot_lo(const uint4& w, const uint4& a, int s) {
  s = dot4(w.x & 0x0F0F0F0Fu, a.x, s);
  s = dot4(w.y & 0x0F0F0F0Fu, a.y, s);
  s = dot4(w.z & 0x0F0F0F0Fu, a.z, s);
  return dot4(w.w & 0x0F0F0F0Fu, a.w, s);
}
// High nibbles without a shift: byte (16*hi) ^ 0x80 is the signed int8
// 16*(hi - 8) (one v_bitop3 per dword), so this returns 16 * sum (hi - 8) * a;
// callers add back 8 * sum a from the activation code sums.
__device__ __forceinline__ int dot_hi16(const uint4& w, const uint4& a, int s) {
  s = dot4((w.x & 0xF0F0F0F0u) ^ 0x80808080u, a.x, s);
  s = dot4((w.y & 0xF0F0F0F0u) ^ 0x80808080u, a.y, s);
  s = dot4((w.z & 0xF0F0F0F0u) ^ 0x80808080u, a.z, s);
  return dot4((w.w & 0xF0F0F0F0u) ^ 0x80808080u, a.w, s);
}
__device__ __forceinline__ int dot_i8(const uint4& w, const uint4& a, int s) {
  s = dot4(w.x, a.x, s);
  s = dot4(w.y, a.y, s);
  s = dot4(w.z, a.z, s);
  return dot4(w.w, a.w, s);
}

// 6-bit scales / mins of sub-blocks 2t and 2t+1 (get_scale_min_k4,
// quant.cpp:356-363).  Lane t of a quad holds header dword t (d1..d3 = scale
// bytes 0-3, 4-7, 8-11).  For t < 2 both sub-blocks are < 4: sc = byte[s] &
// 63, m = byte[s+4] & 63; for t >= 2 they are >= 4 and take their low 4 bits
// from byte[s+4] and their top 2 bits from byte[s-4] / byte[s].  With u = t&1
// every needed byte sits at bit 16u of its dword, so one quad_perm per
// operand fetches the right dword for both halves of the quad:
//   X = t<2 ? d1 : d3 (scales), Y = t<2 ? d2 : d3 (mins),
//   P = d1, Q = d2 (top bits, t >= 2 only; width 0 for t < 2).
struct Q4kLane {  // per-lane field positions, fixed for the whole kernel
  uint32_t sh, w, wh, om;
};
__device__ __forceinline__ Q4kLane q4k_lane(int t) {
  Q4kLane c;
  c.sh = (t & 1) * 16;
  c.w = t < 2 ? 6 : 4;
  c.wh = t < 2 ? 0 : 2;
  c.om = t < 2 ? 0 : 4;
  return c;
}
__device__ __forceinline__ uint32_t bfe(uint32_t v, uint32_t off, uint32_t w) {
  return __builtin_amdgcn_ubfe(v, off, w);
}
template <int CTRL>
__device__ __forceinline__ uint32_t qperm(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ void q4k_scales(const Q4kLane& c, uint32_t h, int& sc0, int& sc1,
                                           int& m0, int& m1) {
  const uint32_t X = qperm<0xF5>(h);  // [1,1,3,3]
  const uint32_t Y = qperm<0xFA>(h);  // [2,2,3,3]
  const uint32_t P = qperm<0x50>(h);  // [0,0,1,1]
  const uint32_t Q = qperm<0xA0>(h);  // [0,0,2,2]
  sc0 = (int)(bfe(X, c.sh, c.w) | (bfe(P, c.sh + 6, c.wh) << 4));
  sc1 = (int)(bfe(X, c.sh + 8, c.w) | (bfe(P, c.sh + 14, c.wh) << 4));
  m0 = (int)(bfe(Y, c.sh + c.om, c.w) | (bfe(Q, c.sh + 6, c.wh) << 4));
  m1 = (int)(bfe(Y, c.sh + 8 + c.om, c.w) | (bfe(Q, c.sh + 14, c.wh) << 4));
}

struct GemvArgs {
  const uint8_t* w;
  size_t nbw;
  const int8_t* qa;
  const float* da;
  const int* sa;
  void* y;
  int M, N, K;
  const void* x;  // raw activations [M, K] (f32 / bf16) for the fused-quantize kernels
};

// Quantized activations of one (token, block) as a lane uses them.
//   Q4_K (lane t of the quad): a0,a1 = codes of sub-block 2t, a2,a3 = codes
//     of sub-block 2t+1, s0/s1 = their code sums, d = Q8_K scale.
//   Q4_0 / Q8_0: a0,a1 = the block's 32 codes, s0 = sum of its first 16
//     codes (Q4_0 only), d = the fp16-rounded Q8_0 scale.
struct AReg {
  uint4 a0, a1, a2, a3;
  int s0, s1;
  float d;
};

template <int QT>
__device__ __forceinline__ void load_a(AReg& x, const GemvArgs& a, int m, int kb, int nbr, int t) {
  const size_t K = (size_t)a.K;
  if constexpr (QT == UB_Q4_K) {
    const uint4* ab = (const uint4*)(a.qa + m * K + (size_t)kb * 256 + 64 * t);
    x.a0 = ab[0];
    x.a1 = ab[1];
    x.a2 = ab[2];
    x.a3 = ab[3];
    const int2 ss = *(const int2*)(a.sa + m * (K >> 5) + (size_t)kb * 8 + 2 * t);
    x.s0 = ss.x;
    x.s1 = ss.y;
  } else {
    const uint4* ap = (const uint4*)(a.qa + m * K + (size_t)kb * 32);
    x.a0 = ap[0];
    x.a1 = ap[1];
    if constexpr (QT == UB_Q4_0) x.s0 = a.sa[(size_t)m * nbr + kb];
  }
  x.d = a.da[(size_t)m * nbr + kb];
}

// ------------------------------------------------------------ GEMV kernel
// A wavefront owns R consecutive rows and issues the loads of U
// block-iterations x R rows before any arithmetic; the activations of those
// blocks are then read once from L1/L2 and reused across the R rows.
//
// XQ = f32 / bf16 (Q4_0 / Q8_0, 1-2 tokens, K <= kFusedMaxK): the workgroup
// first quantizes the raw activations a.x to Q8_0 into LDS itself (the same
// arithmetic as the workspace quantizer, bit-identical codes), so one launch
// does the whole QMatMul.  The raw activations are loaded before the first
// block-iteration's weights, so waiting for them leaves the weights in flight.
constexpr int kFusedMaxK = 8192;
template <int QT, int MT, int R, int U, int OT, int XQ = -1>
__global__ void __launch_bounds__(256) k_gemv(GemvArgs a) {
  using G = Geo<QT>;
  constexpr bool kFused = XQ >= 0;
  static_assert(!kFused || (QT != UB_Q4_K && MT <= 2), "fused quantization: Q4_0 / Q8_0, M <= 2");
  constexpr int kNbMax = kFused ? kFusedMaxK / 32 : 1;
  __shared__ __attribute__((aligned(16))) uint8_t xq_codes[kFused ? MT : 1][kNbMax * 32];
  __shared__ float xq_d[kFused ? MT : 1][kNbMax];
  __shared__ int xq_s[kFused ? MT : 1][kNbMax];
  const int lane = threadIdx.x & 63;
  // wave-uniform (scalar) row index, so the buffer descriptors live in SGPRs
  const int row0 = (blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * R;
  if (!kFused && row0 >= a.N) return;  // (fused: every wave takes part in the quantization)
  const int nbr = a.K / G::BK;
  const int kb0 = lane / G::LPB, t = lane % G::LPB;
  const Q4kLane ql = q4k_lane(t);
  const int M = a.M, N = a.N, K = a.K;
  const int nrows = max(0, min(R, N - row0));
  const __amdgpu_buffer_rsrc_t rq =
      rsrc(a.w + a.nbw * G::HB + (size_t)row0 * nbr * G::QB, (uint32_t)(nrows * nbr * G::QB));
  const __amdgpu_buffer_rsrc_t rh =
      rsrc(a.w + (size_t)row0 * nbr * G::HB, (uint32_t)(nrows * nbr * G::HB));

  float acc[R * MT];
#pragma unroll
  for (int i = 0; i < R * MT; i++) acc[i] = 0.f;

  // Activations of one block-iteration and token: loaded together with the
  // weights when few tokens share the pass (MT <= 2), so one wait covers both;
  // otherwise per token, as the arithmetic reaches it.
  constexpr bool kPre = MT <= 2;
  WReg wr[U][R];
  auto load_wts = [&](int it) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int kb = kb0 + (it + u) * G::BPI;
#pragma unroll
      for (int r = 0; r < R; r++)
        load_w<QT>(wr[u][r], rq, rh, (uint32_t)(r * nbr + kb), kb < nbr, t);
    }
  };
  if constexpr (kFused) {
    // 8 lanes per 32-element block, 4 elements per lane, 32 blocks per pass
    const int tid = threadIdx.x, il = tid & 7;
    constexpr int kPass = kNbMax / 32;
    const int nb = K / 32;
    const __amdgpu_buffer_rsrc_t rx = rsrc_u(a.x, (uint32_t)(M * K * (XQ == UB_F32 ? 4 : 2)));
    uint32_t xr[MT][kPass][XQ == UB_F32 ? 4 : 2];
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
      for (int p = 0; p < kPass; p++) {
        const int b = p * 32 + (tid >> 3);
        const bool ok = (MT == 1 || m < M) && b < nb;
        const uint32_t e = (uint32_t)(m * K + b * 32 + 4 * il);
        if constexpr (XQ == UB_F32) {
          const uint4 v = bload16(rx, ok ? e * 4 : kOOB);
          xr[m][p][0] = v.x; xr[m][p][1] = v.y; xr[m][p][2] = v.z; xr[m][p][3] = v.w;
        } else {
          const uint2 v = bload8(rx, ok ? e * 2 : kOOB);
          xr[m][p][0] = v.x; xr[m][p][1] = v.y;
        }
      }
    load_wts(0);
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
      for (int p = 0; p < kPass; p++) {
        if (p * 32 >= nb || (MT > 1 && m >= M)) continue;  // (uniform) no block of this pass
        const int b = p * 32 + (tid >> 3);
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          if constexpr (XQ == UB_F32) v[j] = __uint_as_float(xr[m][p][j]);
          else v[j] = __uint_as_float((j & 1) ? (xr[m][p][j >> 1] & 0xffff0000u) : (xr[m][p][j >> 1] << 16));
        }
        // Candle / GGML from_float: d = amax / 127 over the block, q = round(x / d)
        float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
        const float d = __fdiv_rn(amax, 127.0f);
        const float id = d != 0.f ? __fdiv_rn(1.0f, d) : 0.f;
        uint32_t pk = 0;
        int sq = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int q = (int)roundf(__fmul_rn(v[j], id));
          pk |= (uint32_t)(q & 0xff) << (8 * j);
          sq += q;
        }
        // sum of the block's first 16 codes (lanes 0-3 of the group)
        sq += __shfl_xor(sq, 1, 64);
        sq += __shfl_xor(sq, 2, 64);
        if (b < nb) {
          *(uint32_t*)&xq_codes[m][b * 32 + 4 * il] = pk;
          if (il == 0) {
            xq_d[m][b] = ub_f16_to_f32(ub_f32_to_f16(d));
            xq_s[m][b] = sq;
          }
        }
      }
    // publish the LDS activations without waiting for the weight loads
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
  for (int it = 0; it * G::BPI < nbr; it += U) {
    AReg ar[kPre ? U : 1][kPre ? MT : 1];
    if (!kFused || it > 0) load_wts(it);
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int kb = kb0 + (it + u) * G::BPI;
      if constexpr (kPre) {
#pragma unroll
        for (int m = 0; m < MT; m++) {
          if (MT == 1 || m < M) {
            if constexpr (kFused) {
              const int kc = min(kb, nbr - 1);
              ar[u][m].a0 = *(const uint4*)&xq_codes[m][kc * 32];
              ar[u][m].a1 = *(const uint4*)&xq_codes[m][kc * 32 + 16];
              ar[u][m].d = xq_d[m][kc];
              ar[u][m].s0 = xq_s[m][kc];
            } else {
              load_a<QT>(ar[u][m], a, m, min(kb, nbr - 1), nbr, t);
            }
          }
        }
      }
    }
    // keep every load of this pass ahead of the arithmetic
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int kb = min(kb0 + (it + u) * G::BPI, nbr - 1);  // clamped: activations stay in bounds
      if constexpr (QT == UB_Q4_K) {
        // Per row: sub-block scales / mins as floats, and d, dmin.  The block
        // sum sc0*slo + sc1*shi (and m0*s0 + m1*s1) is formed in f32, where it
        // is exact: each product has < 24 significant bits and so does the sum
        // (|sc|, |m| < 64, |dot| < 2^16).
        float fsc0[R], fsc1[R], fm0[R], fm1[R], dw[R], dm[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
          const uint32_t hv = wr[u][r].h;
          int sc0, sc1, mn0, mn1;
          q4k_scales(ql, hv, sc0, sc1, mn0, mn1);
          fsc0[r] = (float)sc0;
          fsc1[r] = (float)sc1;
          fm0[r] = (float)mn0;
          fm1[r] = (float)mn1;
          const uint32_t h0 = qperm<0x00>(hv);  // d | dmin << 16
          dw[r] = ub_f16_to_f32((uint16_t)(h0 & 0xffff));
          dm[r] = ub_f16_to_f32((uint16_t)(h0 >> 16));
        }
#pragma unroll
        for (int m = 0; m < MT; m++) {
          if (MT == 1 || m < M) {
            AReg x;
            if constexpr (kPre) x = ar[u][m];
            else load_a<QT>(x, a, m, kb, nbr, t);
            const int s8 = 8 * x.s1;
            const float fs0 = (float)x.s0, fs1 = (float)x.s1;
#pragma unroll
            for (int r = 0; r < R; r++) {
              const int slo = dot_lo(wr[u][r].q1, x.a1, dot_lo(wr[u][r].q0, x.a0, 0));
              const int shi = (dot_hi16(wr[u][r].q1, x.a3, dot_hi16(wr[u][r].q0, x.a2, 0)) >> 4) + s8;
              const float isum = fsc0[r] * (float)slo + fsc1[r] * (float)shi;
              const float imin = fm0[r] * fs0 + fm1[r] * fs1;
              acc[r * MT + m] += (dw[r] * x.d) * isum - (dm[r] * x.d) * imin;
            }
          }
        }
      } else {
#pragma unroll
        for (int m = 0; m < MT; m++) {
          if (MT == 1 || m < M) {
            AReg x;
            if constexpr (kPre) x = ar[u][m];
            else load_a<QT>(x, a, m, kb, nbr, t);
            const int s8 = 8 * x.s0;  // Q4_0: 8 * (sum of the block's first 16 activation codes)
#pragma unroll
            for (int r = 0; r < R; r++) {
              int s;
              if constexpr (QT == UB_Q4_0)
                s = (dot_hi16(wr[u][r].q0, x.a1, 0) >> 4) + dot_lo(wr[u][r].q0, x.a0, 0) - s8;
              else
                s = dot_i8(wr[u][r].q1, x.a1, dot_i8(wr[u][r].q0, x.a0, 0));
              // an out-of-range block reads d = 0 and adds nothing
              acc[r * MT + m] += (float)s * ub_f16_to_f32((uint16_t)wr[u][r].h) * x.d;
            }
          }
        }
      }
    }
  }
  const float v = wave_reduce_scatter<R * MT>(acc, lane);
  constexpr int SH = 6 - ilog2<R * MT>();
  if ((lane & ((1 << SH) - 1)) == 0) {
    const int idx = lane >> SH;
    const int r = idx / MT, m = idx % MT;
    if (m < M && r < nrows) store_out<OT>(a.y, (size_t)m * N + row0 + r, v);
  }
}

// ------------------------------------------- Q4_K GEMV, LDS-staged operands
// The same arithmetic as k_gemv<Q4_K>, with a different load path: each
// wavefront streams its R rows, 16 super-blocks (4096 elements) at a time,
// straight from HBM into its own LDS slice with direct-to-LDS buffer loads
// (buffer_load_dwordx4 ... lds).  Every code load instruction covers 1 KiB of
// contiguous bytes (headers: 256 B per row, or 1 KiB for 4 rows), instead of
// the 32-byte-strided halves the register path needs, and no VGPRs are held
// while the loads are in flight.  The chunk's quantized activations (codes,
// 32-element sums, d) are shared by the workgroup in one LDS region, either
// loaded from the workspace (split over the wavefronts) or computed in place
// from the raw activations.  The block math then reads every operand from
// LDS in the quad-per-block layout.
// LDS: per wavefront R x (2 KiB codes + 256 B headers); per workgroup MT x
// (4 KiB codes + 1 KiB sums and scales).
constexpr int kQ4kCB = 16;  // super-blocks per chunk and row

// vmcnt(0), expcnt / lgkmcnt fields left at their maximum.  The compiler's
// wait insertion does not see direct-to-LDS loads as LDS stores, so reads of
// their data are fenced by hand.
__device__ __forceinline__ void wait_vm() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __builtin_amdgcn_sched_barrier(0);
}

// Q8_K quantization of one chunk (16 super-blocks) of token m into the LDS
// activation layout the block math reads (codes | 32-element sums | d), by
// the whole workgroup of W wavefronts: each block is taken by L = 4W lanes
// (16 / W blocks per wavefront), E = 64 / W consecutive elements per lane.
// Same rule as k_quantize_q8_k (Candle BlockQ8K::from_float): max = the
// signed value of largest |x|, lowest index on a tie; iscale = -128/max;
// q = min(127, round(iscale*x)); d = 1/iscale.  The signed max comes from
// the block's max and min (two L-lane reductions); only when +a and -a both
// reach the largest |x| does the lowest index decide, by a third reduction
// of (index << 1 | sign).  The quantizer runs in every workgroup of the
// one-call kernel, so it is kept to ~10 VALU ops per element.  Lane groups
// of 16 reduce with DPP (partners L^1, L^2, L^7, L^15), 32 and 64 with
// permlane16 / permlane32 swaps.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
// max / min over aligned groups of G lanes (G = 2 .. 64)
template <int G, bool MAXF>
__device__ __forceinline__ uint32_t group_reduce(uint32_t v) {
  auto op = [](uint32_t a, uint32_t b) -> uint32_t {
    if constexpr (MAXF) return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
    else return (uint32_t)min((int)a, (int)b);
  };
  v = op(v, (uint32_t)dpp_i<0xB1>((int)v));
  if constexpr (G >= 4) v = op(v, (uint32_t)dpp_i<0x4E>((int)v));
  if constexpr (G >= 8) v = op(v, (uint32_t)dpp_i<0x141>((int)v));
  if constexpr (G >= 16) v = op(v, (uint32_t)dpp_i<0x140>((int)v));
  if constexpr (G >= 32) {
    auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = op(r[0], r[1]);
  }
  if constexpr (G >= 64) {
    auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    v = op(r[0], r[1]);
  }
  return v;
}
template <int G>
__device__ __forceinline__ int group_sum(int v) {
  v += dpp_i<0xB1>(v);
  if constexpr (G >= 4) v += dpp_i<0x4E>(v);
  if constexpr (G >= 8) v += dpp_i<0x141>(v);
  return v;
}

// Raw activations of one lane's E elements, loaded (as f32 or bf16 bits)
// before the chunk's weight loads are issued, so that waiting for them does
// not also wait for the weights (vector-memory counters retire in order).
template <int W, int XT>
struct XRaw {
  static constexpr int E = 64 / W;
  static constexpr int NW = XT == UB_F32 ? E : E / 2;  // 32-bit words
  uint32_t w[NW];
};
template <int W, int XT>
__device__ __forceinline__ void q8k_load(XRaw<W, XT>& xr, const void* x, int K, int m, int c0,
                                         int nbr, int wv, int lane) {
  constexpr int L = 4 * W, E = 64 / W;
  const int jb = wv * (16 / W) + lane / L, il = lane % L;
  const int blk = min(c0 + jb, nbr - 1);  // blocks past the row are zeroed after the load
  const size_t e0 = (size_t)m * K + (size_t)blk * 256 + il * E;
  const uint32_t* p = (const uint32_t*)x + (XT == UB_F32 ? e0 : e0 / 2);
  if constexpr (XRaw<W, XT>::NW >= 4) {
#pragma unroll
    for (int i = 0; i < XRaw<W, XT>::NW / 4; i++) {
      const uint4 u = ((const uint4*)p)[i];
      xr.w[4 * i] = u.x; xr.w[4 * i + 1] = u.y; xr.w[4 * i + 2] = u.z; xr.w[4 * i + 3] = u.w;
    }
  } else {
    const uint2 u = *(const uint2*)p;
    xr.w[0] = u.x; xr.w[1] = u.y;
  }
}

template <int W, int XT>
__device__ __forceinline__ void q8k_chunk_to_lds(const XRaw<W, XT>& xr, int c0, int nbr,
                                                 uint8_t* am, int wv, int lane) {
  constexpr int L = 4 * W, E = 64 / W;  // lanes per block, elements per lane
  const int jb = wv * (16 / W) + lane / L, il = lane % L;
  const bool in = c0 + jb < nbr;
  float v[E];
#pragma unroll
  for (int j = 0; j < E; j++) {
    uint32_t u;
    if constexpr (XT == UB_F32) u = xr.w[j];
    else u = (j & 1) ? (xr.w[j >> 1] & 0xffff0000u) : (xr.w[j >> 1] << 16);
    v[j] = in ? __uint_as_float(u) : 0.f;
  }
  // Largest |x| with its sign.  The block's max and min decide it unless
  // +a and -a both occur (a = the largest |x|); only then is the lowest
  // index among them needed (rare: that branch costs the old arg-max).
  float hi = v[0], lo = v[0];
#pragma unroll
  for (int j = 1; j < E; j++) {
    hi = fmaxf(hi, v[j]);
    lo = fminf(lo, v[j]);
  }
  hi = __uint_as_float(group_reduce<L, true>(__float_as_uint(hi)));
  lo = -__uint_as_float(group_reduce<L, true>(__float_as_uint(-lo)));
  const float amax = fmaxf(hi, -lo);
  float mx = hi > -lo ? hi : lo;
  if (hi == -lo && amax != 0.f) {  // both signs reach amax: lowest index wins
    int key = 0x7fffffff;
#pragma unroll
    for (int j = E - 1; j >= 0; j--)
      if (fabsf(v[j]) == amax) key = ((il * E + j) << 1) | (int)(__float_as_uint(v[j]) >> 31);
    key = (int)group_reduce<L, false>((uint32_t)key);
    mx = (key & 1) ? -amax : amax;
  }
  uint32_t pk[E / 4];
#pragma unroll
  for (int i = 0; i < E / 4; i++) pk[i] = 0;
  int sum = 0;
  float d = 0.f;
  if (amax != 0.f) {
    // roundf(p) = trunc(p + copysign(0.5 - 2^-25, p)) for every float |p| <= 130
    // (checked exhaustively); the int conversion truncates.  p must be
    // rounded before the add: the empty asm keeps the compiler from
    // contracting the multiply and the add into one fma.
    const float iscale = __fdiv_rn(-128.0f, mx);
    const float kHalf = 0.49999997f;
#pragma unroll
    for (int j = 0; j < E; j++) {
      float pj = __fmul_rn(iscale, v[j]);
      asm("" : "+v"(pj));
      const int q = min((int)__fadd_rn(pj, __builtin_copysignf(kHalf, pj)), 127);
      pk[j >> 2] |= (uint32_t)(q & 0xff) << (8 * (j & 3));
    }
#pragma unroll
    for (int i = 0; i < E / 4; i++) sum = __builtin_amdgcn_sdot4((int)pk[i], 0x01010101, sum, false);
    d = __fdiv_rn(1.0f, iscale);
  }
  // 16-byte unit u of block jb is stored at unit u ^ (jb & 3) (see act_unit)
  const int lb = il * E;
  uint8_t* cp = am + jb * 256 + ((((lb >> 4) ^ (jb & 3)) << 4) | (lb & 15));
  if constexpr (E == 16) *(uint4*)cp = make_uint4(pk[0], pk[1], pk[2], pk[3]);
  else if constexpr (E == 8) *(uint2*)cp = make_uint2(pk[0], pk[1]);
  else *(uint32_t*)cp = pk[0];
  constexpr int LS = 32 / E;  // lanes per 32-element sub-block
  sum = group_sum<LS>(sum);
  if (il % LS == 0) *(int*)(am + 4096 + (jb * 8 + il / LS) * 4) = sum;
  if (il == 0) *(float*)(am + 4096 + 512 + jb * 4) = d;
}

// Direct-to-LDS buffer loads: lane i's 16 (4) bytes land at lds + 16i (4i);
// the global address must be aligned to the access size.
template <int AUX>
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16,
                                           off, 0, 0, AUX);
}
template <int AUX>
__device__ __forceinline__ void lds_load4(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 4,
                                           off, 0, 0, AUX);
}

// W wavefronts per workgroup, R rows per wavefront, MT tokens.  XQ < 0:
// quantized activations come from the workspace; XQ = f32 / bf16: the
// kernel quantizes the raw activations a.x itself, per workgroup and chunk,
// while its weight loads are in flight (no separate quantize launch).
// Wait until at most 3n vector-memory ops are outstanding: the loads of the
// last n rows (three per row, issued last) may still be in flight.
__device__ __forceinline__ void wait_vm_rows(int n) {
  __builtin_amdgcn_sched_barrier(0);
  switch (n) {  // immediates: vmcnt(3n), expcnt / lgkmcnt at their maximum
    case 0: __builtin_amdgcn_s_waitcnt(0x0F70); break;
    case 1: __builtin_amdgcn_s_waitcnt(0x0F73); break;
    case 2: __builtin_amdgcn_s_waitcnt(0x0F76); break;
    default: __builtin_amdgcn_s_waitcnt(0x0F79); break;
  }
  __builtin_amdgcn_sched_barrier(0);
}

template <int W, int MT, int R, int OT, int XQ>
__global__ void __launch_bounds__(64 * W) k_gemv_q4k_lds(GemvArgs a) {
  constexpr int kRowB = kQ4kCB * 128 + kQ4kCB * 16;  // one row's chunk: codes, then headers
  constexpr int kActB = 4096 + 1024;  // per token: codes, then sums (512 B) + d (64 B)
  // One LDS object per row slot (each holding that row of every wave) and one
  // for the activations: the compiler tracks direct-to-LDS loads per object,
  // so reading row r waits only for row r's loads, and the activation writes
  // do not wait for the weights.
  __shared__ __attribute__((aligned(16))) uint8_t lds_r0[W * kRowB];
  __shared__ __attribute__((aligned(16))) uint8_t lds_r1[R > 1 ? W * kRowB : 16];
  __shared__ __attribute__((aligned(16))) uint8_t lds_r2[R > 2 ? W * kRowB : 16];
  __shared__ __attribute__((aligned(16))) uint8_t lds_r3[R > 3 ? W * kRowB : 16];
  __shared__ __attribute__((aligned(16))) uint8_t lds_act[MT * kActB];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = (blockIdx.x * W + wv) * R;
  const int nbr = a.K / 256;
  const int M = a.M, N = a.N;
  const int nrows = max(0, min(R, N - row0));  // 0: this wave only helps with activations
  const __amdgpu_buffer_rsrc_t rq = rsrc_u(a.w + a.nbw * 16 + (size_t)min(row0, N) * nbr * 128,
                                           (uint32_t)(nrows * nbr * 128));
  const __amdgpu_buffer_rsrc_t rh =
      rsrc_u(a.w + (size_t)min(row0, N) * nbr * 16, (uint32_t)(nrows * nbr * 16));
  // one descriptor over the activation workspace: codes | d | sums
  const uint8_t* qa = (const uint8_t*)a.qa;
  const uint32_t off_d = (uint32_t)((const uint8_t*)a.da - qa);
  const uint32_t off_s = (uint32_t)((const uint8_t*)a.sa - qa);
  const int nact = min(M, MT);
  const __amdgpu_buffer_rsrc_t ra = rsrc_u(qa, off_s + (uint32_t)(nact * (a.K / 32) * 4));
  // this wave's slice of row slot r: 2 KiB of codes, then 256 B of headers
  auto row_lds = [&](int r) -> uint8_t* {
    uint8_t* base = r == 0 ? lds_r0 : r == 1 ? lds_r1 : r == 2 ? lds_r2 : lds_r3;
    return base + wv * kRowB;
  };
  uint8_t* al = lds_act;
  const int kb = lane >> 2, t = lane & 3;
  const Q4kLane ql = q4k_lane(t);

  float acc[R * MT];
#pragma unroll
  for (int i = 0; i < R * MT; i++) acc[i] = 0.f;

  for (int c0 = 0; c0 < nbr; c0 += kQ4kCB) {
    if (c0 > 0) __syncthreads();  // every wave is done with the previous chunk's activations
    XRaw<W, (XQ < 0 ? UB_F32 : XQ)> xr[XQ >= 0 ? MT : 1];
    if constexpr (XQ >= 0) {
#pragma unroll
      for (int m = 0; m < MT; m++)
        if (MT == 1 || m < M) q8k_load<W, XQ>(xr[m], a.x, a.K, m, c0, nbr, wv, lane);
    }
    // activations (issued before the weights, so that waiting for them leaves
    // the weights in flight): per token 4 x 1 KiB of codes + one instruction for the
    // sums (lanes 0-31) and d (lanes 32-35); instruction i goes to wave i % W
#pragma unroll
    for (int i = 0; i < (XQ < 0 ? 5 * MT : 0); i++) {
      if (i % W != wv) continue;
      const int m = i / 5, j = i % 5;
      if (MT > 1 && m >= M) continue;
      uint32_t off;
      if (j < 4) {
        // LDS unit P = 64 j + lane holds logical unit (P & 15) ^ (kb & 3) of
        // block kb = P >> 4 (the bank swizzle of the activation codes)
        const int P = j * 64 + lane, kbp = P >> 4;
        const uint32_t e = (uint32_t)c0 * 256 + kbp * 256 + (((P & 15) ^ (kbp & 3)) << 4);  // element in the row
        off = e < (uint32_t)a.K ? (uint32_t)(m * a.K) + e : kOOB;
      } else if (lane < 32) {
        const uint32_t e = (uint32_t)c0 * 8 + lane * 4;  // 32-element sum index in the row
        off = e < (uint32_t)(a.K / 32) ? off_s + (m * (a.K / 32) + e) * 4 : kOOB;
      } else {
        const uint32_t e = (uint32_t)c0 + (lane - 32) * 4;  // block index in the row
        off = lane < 36 && e < (uint32_t)nbr ? off_d + (m * nbr + e) * 4 : kOOB;
      }
      lds_load16<0>(ra, al + m * kActB + j * 1024, off);
    }
    // weights, row by row (the block math waits for one row at a time):
    // 16 headers (256 B, 4 B per lane), then codes [c0*128, c0*128 + 2048) in
    // two 1 KiB instructions
    const uint32_t rowb = (uint32_t)nbr * 128;
#pragma unroll
    for (int r = 0; r < R; r++) {
      uint8_t* rl = row_lds(r);
      const uint32_t in_hdr = (uint32_t)c0 * 16 + lane * 4;
      lds_load4<kAuxNT>(rh, rl + 2048, in_hdr < (uint32_t)nbr * 16 ? r * nbr * 16 + in_hdr : kOOB);
#pragma unroll
      for (int h = 0; h < 2; h++) {
        // LDS unit P = 64 h + lane holds logical unit (P & 7) ^ ((kb >> 1) & 1)
        // of super-block kb = P >> 3 (the bank swizzle of the weight codes)
        const int P = h * 64 + lane, kbp = P >> 3;
        const uint32_t in_row = (uint32_t)c0 * 128 + kbp * 128 + (((P & 7) ^ ((kbp >> 1) & 1)) << 4);
        lds_load16<kAuxNT>(rq, rl + h * 1024, in_row < rowb ? r * rowb + in_row : kOOB);
      }
    }
    if constexpr (XQ >= 0) {
#pragma unroll
      for (int m = 0; m < MT; m++)
        if (MT == 1 || m < M) q8k_chunk_to_lds<W, XQ>(xr[m], c0, nbr, al + m * kActB, wv, lane);
    }
    // Activations of every wave in LDS, then this wave's weights.  A plain
    // s_barrier after waiting for just the activations (own LDS writes:
    // lgkmcnt(0); own activation DMA: vmcnt(#weight loads), as the counter
    // retires in order) -- __syncthreads() would also wait for the weight
    // loads still in flight.  The empty asm with a memory clobber keeps the
    // compiler from moving LDS accesses across the barrier.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XQ >= 0) {
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    } else if constexpr (R == 4) {
      __builtin_amdgcn_s_waitcnt(0x0F7C);  // vmcnt(12): the 12 weight loads may be in flight
    } else if constexpr (R == 2) {
      __builtin_amdgcn_s_waitcnt(0x0F76);  // vmcnt(6)
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F73);  // vmcnt(3)
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    if (nrows > 0) {
      const bool ok = c0 + kb < nbr;
      AReg x[MT];
#pragma unroll
      for (int m = 0; m < MT; m++) {
        if (MT == 1 || m < M) {
          const uint8_t* am = al + m * kActB;
          // the lane's four units 4t..4t+3 of block kb, swizzled: lanes of
          // one 16-lane LDS pass (kb = 0..3) then hit distinct banks
          const uint8_t* ab = am + kb * 256;
          const int sw = kb & 3;
          x[m].a0 = *(const uint4*)(ab + (((4 * t) ^ sw) << 4));
          x[m].a1 = *(const uint4*)(ab + (((4 * t + 1) ^ sw) << 4));
          x[m].a2 = *(const uint4*)(ab + (((4 * t + 2) ^ sw) << 4));
          x[m].a3 = *(const uint4*)(ab + (((4 * t + 3) ^ sw) << 4));
          const int2 ss = *(const int2*)(am + 4096 + (kb * 8 + 2 * t) * 4);
          x[m].s0 = ss.x;
          x[m].s1 = ss.y;
          x[m].d = *(const float*)(am + 4096 + 512 + kb * 4);
        }
      }
      // row by row, each as soon as its own two code loads have landed
#pragma unroll
      for (int r = 0; r < R; r++) {
        wait_vm_rows(R - 1 - r);
        const uint8_t* rl = row_lds(r);
        const uint32_t hv = *(const uint32_t*)(rl + 2048 + kb * 16 + t * 4);
        const int wsw = (kb >> 1) & 1;  // weight-code swizzle of super-block kb
        const uint4 q0 = *(const uint4*)(rl + kb * 128 + (((2 * t) ^ wsw) << 4));
        const uint4 q1 = *(const uint4*)(rl + kb * 128 + (((2 * t + 1) ^ wsw) << 4));
        int sc0, sc1, mn0, mn1;
        q4k_scales(ql, hv, sc0, sc1, mn0, mn1);
        const float fsc0 = (float)sc0, fsc1 = (float)sc1, fm0 = (float)mn0, fm1 = (float)mn1;
        const uint32_t h0 = qperm<0x00>(hv);  // d | dmin << 16
        const float dw = ok ? ub_f16_to_f32((uint16_t)(h0 & 0xffff)) : 0.f;
        const float dm = ok ? ub_f16_to_f32((uint16_t)(h0 >> 16)) : 0.f;
#pragma unroll
        for (int m = 0; m < MT; m++) {
          if (MT == 1 || m < M) {
            const int slo = dot_lo(q1, x[m].a1, dot_lo(q0, x[m].a0, 0));
            const int shi = (dot_hi16(q1, x[m].a3, dot_hi16(q0, x[m].a2, 0)) >> 4) + 8 * x[m].s1;
            const float isum = fsc0 * (float)slo + fsc1 * (float)shi;
            const float imin = fm0 * (float)x[m].s0 + fm1 * (float)x[m].s1;
            acc[r * MT + m] += (dw * x[m].d) * isum - (dm * x[m].d) * imin;
          }
        }
      }
    }
  }
  if (nrows == 0) {  // its out-of-range weight loads still write its slices
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    return;
  }
  const float v = wave_reduce_scatter<R * MT>(acc, lane);
  constexpr int SH = 6 - ilog2<R * MT>();
  if ((lane & ((1 << SH) - 1)) == 0) {
    const int idx = lane >> SH;
    const int r = idx / MT, m = idx % MT;
    if (m < M && r < nrows) store_out<OT>(a.y, (size_t)m * N + row0 + r, v);
  }
}


// ------------------------------------- persistent one-launch Q4_K GEMV
// The block math and LDS layout of k_gemv_q4k_lds (fused activation
// quantization, 1-2 tokens), with a grid sized to the GPU's resident
// capacity: each workgroup quantizes the activations once -- every chunk of
// the row, NCH x 16 super-blocks per token, kept in LDS -- and then loops
// over row groups blockIdx.x, blockIdx.x + gridDim.x, ...  The first row
// group's weight loads are issued before the quantization, which they hide.
// The one-shot kernel repeats the quantization in each of its N / (W R)
// workgroups; here it runs once per resident workgroup.  ROLL: a wave issues
// row r of its next (row group, chunk) unit as soon as its reads of row r
// of the current one have returned, so R rows stay in flight through the
// math (without it the next unit's loads go out after all of the math).
template <int W, int MT, int R, int OT, int XQ, int NCH, bool ROLL>
__global__ void __launch_bounds__(64 * W) k_gemv_q4k_pq(GemvArgs a) {
  constexpr int kRowB = kQ4kCB * 128 + kQ4kCB * 16;
  constexpr int kActB = 4096 + 1024;
  __shared__ __attribute__((aligned(16))) uint8_t lds_r0[W * kRowB];
  __shared__ __attribute__((aligned(16))) uint8_t lds_r1[R > 1 ? W * kRowB : 16];
  __shared__ __attribute__((aligned(16))) uint8_t lds_r2[R > 2 ? W * kRowB : 16];
  __shared__ __attribute__((aligned(16))) uint8_t lds_r3[R > 3 ? W * kRowB : 16];
  __shared__ __attribute__((aligned(16))) uint8_t lds_act[MT * NCH * kActB];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nbr = a.K / 256;
  const int M = a.M, N = a.N;
  const int nrg = (N + W * R - 1) / (W * R);
  auto row_lds = [&](int r) -> uint8_t* {
    uint8_t* base = r == 0 ? lds_r0 : r == 1 ? lds_r1 : r == 2 ? lds_r2 : lds_r3;
    return base + wv * kRowB;
  };
  const int kb = lane >> 2, t = lane & 3;
  const Q4kLane ql = q4k_lane(t);
  const uint32_t rowb = (uint32_t)nbr * 128;
  // weight loads of rows row0.. (nrows of them) for the chunk at c0
  auto issue_rows = [&](int row0, int nrows, int c0) {
    const __amdgpu_buffer_rsrc_t rq = rsrc_u(a.w + a.nbw * 16 + (size_t)min(row0, N) * nbr * 128,
                                             (uint32_t)(nrows * nbr * 128));
    const __amdgpu_buffer_rsrc_t rh =
        rsrc_u(a.w + (size_t)min(row0, N) * nbr * 16, (uint32_t)(nrows * nbr * 16));
#pragma unroll
    for (int r = 0; r < R; r++) {
      uint8_t* rl = row_lds(r);
      const uint32_t in_hdr = (uint32_t)c0 * 16 + lane * 4;
      lds_load4<kAuxNT>(rh, rl + 2048, in_hdr < (uint32_t)nbr * 16 ? r * nbr * 16 + in_hdr : kOOB);
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int P = h * 64 + lane, kbp = P >> 3;
        const uint32_t in_row = (uint32_t)c0 * 128 + kbp * 128 + (((P & 7) ^ ((kbp >> 1) & 1)) << 4);
        lds_load16<kAuxNT>(rq, rl + h * 1024, in_row < rowb ? r * rowb + in_row : kOOB);
      }
    }
  };
  auto rows_of = [&](int rg) { return max(0, min(R, N - (rg * W + wv) * R)); };
  // row r alone (as issue_rows does it for every row)
  auto issue_row = [&](int row0, int nrows, int c0, int r) {
    const __amdgpu_buffer_rsrc_t rq = rsrc_u(a.w + a.nbw * 16 + (size_t)min(row0, N) * nbr * 128,
                                             (uint32_t)(nrows * nbr * 128));
    const __amdgpu_buffer_rsrc_t rh =
        rsrc_u(a.w + (size_t)min(row0, N) * nbr * 16, (uint32_t)(nrows * nbr * 16));
    uint8_t* rl = row_lds(r);
    const uint32_t in_hdr = (uint32_t)c0 * 16 + lane * 4;
    lds_load4<kAuxNT>(rh, rl + 2048, in_hdr < (uint32_t)nbr * 16 ? r * nbr * 16 + in_hdr : kOOB);
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int P = h * 64 + lane, kbp = P >> 3;
      const uint32_t in_row = (uint32_t)c0 * 128 + kbp * 128 + (((P & 7) ^ ((kbp >> 1) & 1)) << 4);
      lds_load16<kAuxNT>(rq, rl + h * 1024, in_row < rowb ? r * rowb + in_row : kOOB);
    }
  };
  // the lane's activation units of chunk c0 (LDS)
  auto load_act = [&](AReg* x, int c0) {
#pragma unroll
    for (int m = 0; m < MT; m++) {
      if (MT == 1 || m < M) {
        const uint8_t* am = lds_act + (m * NCH + c0 / kQ4kCB) * kActB;
        const uint8_t* ab = am + kb * 256;
        const int sw = kb & 3;
        x[m].a0 = *(const uint4*)(ab + (((4 * t) ^ sw) << 4));
        x[m].a1 = *(const uint4*)(ab + (((4 * t + 1) ^ sw) << 4));
        x[m].a2 = *(const uint4*)(ab + (((4 * t + 2) ^ sw) << 4));
        x[m].a3 = *(const uint4*)(ab + (((4 * t + 3) ^ sw) << 4));
        const int2 ss = *(const int2*)(am + 4096 + (kb * 8 + 2 * t) * 4);
        x[m].s0 = ss.x;
        x[m].s1 = ss.y;
        x[m].d = *(const float*)(am + 4096 + 512 + kb * 4);
      }
    }
  };
  struct RowQ {
    uint32_t hv;
    uint4 q0, q1;
  };
  auto read_row = [&](int r) {
    const uint8_t* rl = row_lds(r);
    RowQ q;
    q.hv = *(const uint32_t*)(rl + 2048 + kb * 16 + t * 4);
    const int wsw = (kb >> 1) & 1;  // weight-code swizzle of super-block kb
    q.q0 = *(const uint4*)(rl + kb * 128 + (((2 * t) ^ wsw) << 4));
    q.q1 = *(const uint4*)(rl + kb * 128 + (((2 * t + 1) ^ wsw) << 4));
    return q;
  };
  auto row_math = [&](const RowQ& q, const AReg* x, float* acc, int r, bool ok) {
    int sc0, sc1, mn0, mn1;
    q4k_scales(ql, q.hv, sc0, sc1, mn0, mn1);
    const float fsc0 = (float)sc0, fsc1 = (float)sc1, fm0 = (float)mn0, fm1 = (float)mn1;
    const uint32_t h0 = qperm<0x00>(q.hv);  // d | dmin << 16
    const float dw = ok ? ub_f16_to_f32((uint16_t)(h0 & 0xffff)) : 0.f;
    const float dm = ok ? ub_f16_to_f32((uint16_t)(h0 >> 16)) : 0.f;
#pragma unroll
    for (int m = 0; m < MT; m++) {
      if (MT == 1 || m < M) {
        const int slo = dot_lo(q.q1, x[m].a1, dot_lo(q.q0, x[m].a0, 0));
        const int shi = (dot_hi16(q.q1, x[m].a3, dot_hi16(q.q0, x[m].a2, 0)) >> 4) + 8 * x[m].s1;
        const float isum = fsc0 * (float)slo + fsc1 * (float)shi;
        const float imin = fm0 * (float)x[m].s0 + fm1 * (float)x[m].s1;
        acc[r * MT + m] += (dw * x[m].d) * isum - (dm * x[m].d) * imin;
      }
    }
  };
  auto store_rows = [&](float (&acc)[R * MT], int row0, int nrows) {
    const float v = wave_reduce_scatter<R * MT>(acc, lane);
    constexpr int SH = 6 - ilog2<R * MT>();
    if ((lane & ((1 << SH) - 1)) == 0) {
      const int idx = lane >> SH;
      const int r = idx / MT, m = idx % MT;
      if (m < M && r < nrows) store_out<OT>(a.y, (size_t)m * N + row0 + r, v);
    }
  };

  // ---- raw activations of every chunk, then the first row group's loads,
  // then the quantization (the x loads retire first: counters are in order)
  XRaw<W, XQ> xr[MT][NCH];
#pragma unroll
  for (int m = 0; m < MT; m++)
#pragma unroll
    for (int c = 0; c < NCH; c++)
      if ((MT == 1 || m < M) && c * kQ4kCB < nbr) q8k_load<W, XQ>(xr[m][c], a.x, a.K, m, c * kQ4kCB, nbr, wv, lane);
  int rg = blockIdx.x;
  if (rg < nrg) issue_rows((rg * W + wv) * R, rows_of(rg), 0);
#pragma unroll
  for (int m = 0; m < MT; m++)
#pragma unroll
    for (int c = 0; c < NCH; c++)
      if ((MT == 1 || m < M) && c * kQ4kCB < nbr)
        q8k_chunk_to_lds<W, XQ>(xr[m][c], c * kQ4kCB, nbr, lds_act + (m * NCH + c) * kActB, wv, lane);
  // activations of every wave in LDS; the weight loads stay in flight
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  if constexpr (!ROLL) {
  // one chunk per row: the activation registers serve every row group (an
  // LDS read after the issue would also make the compiler drain the new
  // weight loads before row 0's math)
  AReg x[MT];
  if constexpr (NCH == 1) load_act(x, 0);
  for (bool first = true; rg < nrg; rg += gridDim.x, first = false) {
    const int row0 = (rg * W + wv) * R;
    const int nrows = rows_of(rg);
    float acc[R * MT];
#pragma unroll
    for (int i = 0; i < R * MT; i++) acc[i] = 0.f;
    for (int c0 = 0; c0 < nbr; c0 += kQ4kCB) {
      if (!first || c0 > 0) {
        // this wave's earlier LDS reads of its slices have returned
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_sched_barrier(0);
        issue_rows(row0, nrows, c0);
      }
      if (nrows == 0) continue;
      const bool ok = c0 + kb < nbr;
      if constexpr (NCH > 1) load_act(x, c0);
#pragma unroll
      for (int r = 0; r < R; r++) {
        wait_vm_rows(R - 1 - r);
        RowQ q = read_row(r);
        row_math(q, x, acc, r, ok);
      }
    }
    if (nrows == 0) continue;
    store_rows(acc, row0, nrows);
  }
  // out-of-range loads of a wave without rows still write its slices
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  } else {
  // Rolling prefetch: as soon as this wave's LDS reads of row r of the
  // current (row group, chunk) unit have returned, row r of the next unit
  // is issued into the same slice, so the weight loads stay in flight while
  // the row's math runs.  Loads issued after row r of a unit: rows r+1..R-1
  // of the unit and rows 0..r-1 of the next one, R - 1 rows of three loads
  // each.  After the last unit the "next" rows are issued all the same,
  // out of range (no memory traffic; they write zeros into the slices): no
  // branch around a load, which would make the compiler drain every load
  // at the join.
  float acc[R * MT];
#pragma unroll
  for (int i = 0; i < R * MT; i++) acc[i] = 0.f;
  // one chunk per row: the activation registers are the same for every
  // unit, read once (an LDS read inside the loop would also make the
  // compiler drain the pending weight loads first)
  AReg x[MT];
  if constexpr (NCH == 1) load_act(x, 0);
  for (int c0 = 0; rg < nrg;) {
    const int row0 = (rg * W + wv) * R;
    const int nrows = rows_of(rg);
    int nrg_ = rg, nc0 = c0 + kQ4kCB;
    if (nc0 >= nbr) {
      nc0 = 0;
      nrg_ = rg + gridDim.x;
    }
    const bool has_next = nrg_ < nrg;
    if (nrows > 0) {
      const int nrow0 = (nrg_ * W + wv) * R, nnrows = has_next ? rows_of(nrg_) : 0;
      const bool ok = c0 + kb < nbr;
      if constexpr (NCH > 1) load_act(x, c0);
#pragma unroll
      for (int r = 0; r < R; r++) {
        wait_vm_rows(R - 1);
        RowQ q = read_row(r);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the slice is read
        __builtin_amdgcn_sched_barrier(0);
        issue_row(nrow0, nnrows, nc0, r);
        row_math(q, x, acc, r, ok);
      }
      if (nc0 == 0) {  // the row group is complete
        store_rows(acc, row0, nrows);
#pragma unroll
        for (int i = 0; i < R * MT; i++) acc[i] = 0.f;
      }
    }
    rg = nrg_;
    c0 = nc0;
  }
  // out-of-range loads of a wave without rows still write its slices
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  }
}


// ------------------------------- Q4_0 / Q8_0 one-launch GEMV, LDS-staged
// The load path and grid of k_gemv_q4k_pq for the 32-element formats, with
// the activations quantized to Q8_0 (Candle BlockQ8_0::from_float: d = amax
// / 127, q = round(x / d), d kept as fp16) once per workgroup into LDS.  A
// chunk is 4096 elements = 128 blocks of a row: headers (128 x fp16, 256 B)
// and codes (2 KiB Q4_0, 4 KiB Q8_0) travel HBM -> LDS by direct-to-LDS
// loads, 1 KiB of contiguous bytes per instruction.  Lane (kb = lane / 4,
// t = lane % 4) takes blocks 8 kb + 2t and 8 kb + 2t + 1 of the chunk.
// Activation LDS per token and chunk: codes (4 KiB, 16-byte unit u of
// 256-byte group g at u ^ (g & 3)), then d[128] (f32 of the fp16 scale),
// then s[128] (sum of each block's first 16 codes: the Q4_0 offset term).
template <int QT>
struct Q80Geo {
  static constexpr int QCB = QT == UB_Q8_0 ? 4096 : 2048;  // code bytes per row and chunk
  static constexpr int RowB = QCB + 256;
  static constexpr int PR = QCB / 1024 + 1;  // load instructions per row and chunk
};

// vmcnt(n * PR): the loads of the last n rows (issued last) may be in flight
template <int PR>
__device__ __forceinline__ void wait_vm_rows_pr(int n) {
  __builtin_amdgcn_sched_barrier(0);
  switch (n) {
    case 0: ub_wait_vmcnt<0>(); break;
    case 1: ub_wait_vmcnt<PR>(); break;
    case 2: ub_wait_vmcnt<2 * PR>(); break;
    default: ub_wait_vmcnt<3 * PR>(); break;
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Q8_0 quantization of one 4096-element chunk of token m (W wavefronts, E =
// 64 / W elements per lane, 32 / E lanes per block) into the LDS layout
// above; the same arithmetic as the workspace quantizer.
template <int W, int XT>
__device__ __forceinline__ void q80_chunk_to_lds(const XRaw<W, XT>& xr, int c0b, int nb,
                                                 uint8_t* am, int wv, int lane) {
  constexpr int E = 64 / W, L = 32 / E;
  const int e0 = (wv * 64 + lane) * E;  // first element in the chunk
  const int blk = e0 / 32;
  const bool in = c0b + blk < nb;
  float v[E];
#pragma unroll
  for (int j = 0; j < E; j++) {
    uint32_t u;
    if constexpr (XT == UB_F32) u = xr.w[j];
    else u = (j & 1) ? (xr.w[j >> 1] & 0xffff0000u) : (xr.w[j >> 1] << 16);
    v[j] = in ? __uint_as_float(u) : 0.f;
  }
  float amax = fabsf(v[0]);
#pragma unroll
  for (int j = 1; j < E; j++) amax = fmaxf(amax, fabsf(v[j]));
  if constexpr (L >= 2) amax = fmaxf(amax, __uint_as_float((uint32_t)dpp_i<0xB1>((int)__float_as_uint(amax))));
  if constexpr (L >= 4) amax = fmaxf(amax, __uint_as_float((uint32_t)dpp_i<0x4E>((int)__float_as_uint(amax))));
  const float d = __fdiv_rn(amax, 127.0f);
  const float id = d != 0.f ? __fdiv_rn(1.0f, d) : 0.f;
  uint32_t pk[E / 4];
  int sq = 0;
#pragma unroll
  for (int i = 0; i < E / 4; i++) {
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int q = (int)roundf(__fmul_rn(v[4 * i + j], id));
      w |= (uint32_t)(q & 0xff) << (8 * j);
      if (((e0 + 4 * i + j) & 31) < 16) sq += q;
    }
    pk[i] = w;
  }
  // the block's first-16 sum: lanes holding its first 16 elements
  if constexpr (L == 4) sq += dpp_i<0xB1>(sq);
  const int g = e0 >> 8, u = (e0 >> 4) & 15;
  uint8_t* cp = am + g * 256 + (((u ^ (g & 3)) << 4) | (e0 & 15));
  if constexpr (E == 16) *(uint4*)cp = make_uint4(pk[0], pk[1], pk[2], pk[3]);
  else *(uint2*)cp = make_uint2(pk[0], pk[1]);
  if ((e0 & 31) == 0) {
    *(float*)(am + 4096 + blk * 4) = ub_f16_to_f32(ub_f32_to_f16(d));
    *(int*)(am + 4608 + blk * 4) = sq;
  }
}

template <int QT, int W, int MT, int R, int OT, int XQ, int NCH, bool ROLL>
__global__ void __launch_bounds__(64 * W) k_gemv_q80_pq(GemvArgs a) {
  using G = Q80Geo<QT>;
  constexpr int kActB = 5120;
  static_assert(W == 4 || W == 8, "4 or 8 wavefronts");
  __shared__ __attribute__((aligned(16))) uint8_t lds_r0[W * G::RowB];
  __shared__ __attribute__((aligned(16))) uint8_t lds_r1[R > 1 ? W * G::RowB : 16];
  __shared__ __attribute__((aligned(16))) uint8_t lds_r2[R > 2 ? W * G::RowB : 16];
  __shared__ __attribute__((aligned(16))) uint8_t lds_r3[R > 3 ? W * G::RowB : 16];
  __shared__ __attribute__((aligned(16))) uint8_t lds_act[MT * NCH * kActB];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nb = a.K / 32;  // blocks per row
  const int M = a.M, N = a.N;
  const int nrg = (N + W * R - 1) / (W * R);
  auto row_lds = [&](int r) -> uint8_t* {
    uint8_t* base = r == 0 ? lds_r0 : r == 1 ? lds_r1 : r == 2 ? lds_r2 : lds_r3;
    return base + wv * G::RowB;
  };
  const int kb = lane >> 2, t = lane & 3;
  constexpr int QB = QT == UB_Q8_0 ? 32 : 16;
  const uint32_t rowq = (uint32_t)nb * QB, rowh = (uint32_t)nb * 2;
  // weight loads of rows row0.. for the chunk of blocks c0b..c0b + 127
  auto issue_rows = [&](int row0, int nrows, int c0b) {
    const __amdgpu_buffer_rsrc_t rq = rsrc_u(a.w + a.nbw * 2 + (size_t)min(row0, N) * rowq,
                                             (uint32_t)(nrows * rowq));
    const __amdgpu_buffer_rsrc_t rh =
        rsrc_u(a.w + (size_t)min(row0, N) * rowh, (uint32_t)(nrows * rowh));
#pragma unroll
    for (int r = 0; r < R; r++) {
      uint8_t* rl = row_lds(r);
      const uint32_t in_hdr = (uint32_t)c0b * 2 + lane * 4;
      lds_load4<kAuxNT>(rh, rl + G::QCB, in_hdr < rowh ? r * rowh + in_hdr : kOOB);
#pragma unroll
      for (int h = 0; h < G::QCB / 1024; h++) {
        const int P = h * 64 + lane;
        uint32_t in_row;
        if constexpr (QT == UB_Q4_0) {  // 8 units per 128-byte group, swizzled by group bit 1
          const int g = P >> 3;
          in_row = (uint32_t)c0b * 16 + g * 128 + (((P & 7) ^ ((g >> 1) & 1)) << 4);
        } else {  // 16 units per 256-byte group, swizzled by group bits 0-1
          const int g = P >> 4;
          in_row = (uint32_t)c0b * 32 + g * 256 + (((P & 15) ^ (g & 3)) << 4);
        }
        lds_load16<kAuxNT>(rq, rl + h * 1024, in_row < rowq ? r * rowq + in_row : kOOB);
      }
    }
  };
  auto rows_of = [&](int rg) { return max(0, min(R, N - (rg * W + wv) * R)); };

  // ---- raw activations, the first row group's loads, then the quantization
  XRaw<W, XQ> xr[MT][NCH];
  constexpr int E = 64 / W;
#pragma unroll
  for (int m = 0; m < MT; m++)
#pragma unroll
    for (int c = 0; c < NCH; c++) {
      if ((MT == 1 || m < M) && c * 128 < nb) {
        const int e = min(c * 4096 + (wv * 64 + lane) * E, a.K - E);  // past K: zeroed later
        const uint32_t* p = (const uint32_t*)a.x + (XQ == UB_F32 ? (size_t)m * a.K + e : ((size_t)m * a.K + e) / 2);
#pragma unroll
        for (int i = 0; i < XRaw<W, XQ>::NW / 4; i++) {
          const uint4 u = ((const uint4*)p)[i];
          xr[m][c].w[4 * i] = u.x; xr[m][c].w[4 * i + 1] = u.y;
          xr[m][c].w[4 * i + 2] = u.z; xr[m][c].w[4 * i + 3] = u.w;
        }
        if constexpr (XRaw<W, XQ>::NW == 2) {
          const uint2 u = *(const uint2*)p;
          xr[m][c].w[0] = u.x; xr[m][c].w[1] = u.y;
        }
      }
    }
  int rg = blockIdx.x;
  if (rg < nrg) issue_rows((rg * W + wv) * R, rows_of(rg), 0);
#pragma unroll
  for (int m = 0; m < MT; m++)
#pragma unroll
    for (int c = 0; c < NCH; c++)
      if ((MT == 1 || m < M) && c * 128 < nb)
        q80_chunk_to_lds<W, XQ>(xr[m][c], c * 128, nb, lds_act + (m * NCH + c) * kActB, wv, lane);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's activation writes
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  if constexpr (ROLL) {
    // Rolling prefetch, as in k_gemv_q4k_pq: row r of the next (row group,
    // chunk) unit is issued as soon as this wave's reads of row r of the
    // current one have returned (out of range after the last unit), so
    // every wait leaves R - 1 rows in flight.
    auto issue_row = [&](int row0, int nrows, int c0b, int r) {
      const __amdgpu_buffer_rsrc_t rq = rsrc_u(a.w + a.nbw * 2 + (size_t)min(row0, N) * rowq,
                                               (uint32_t)(nrows * rowq));
      const __amdgpu_buffer_rsrc_t rh =
          rsrc_u(a.w + (size_t)min(row0, N) * rowh, (uint32_t)(nrows * rowh));
      uint8_t* rl = row_lds(r);
      const uint32_t in_hdr = (uint32_t)c0b * 2 + lane * 4;
      lds_load4<kAuxNT>(rh, rl + G::QCB, in_hdr < rowh ? r * rowh + in_hdr : kOOB);
#pragma unroll
      for (int h = 0; h < G::QCB / 1024; h++) {
        const int P = h * 64 + lane;
        uint32_t in_row;
        if constexpr (QT == UB_Q4_0) {
          const int g = P >> 3;
          in_row = (uint32_t)c0b * 16 + g * 128 + (((P & 7) ^ ((g >> 1) & 1)) << 4);
        } else {
          const int g = P >> 4;
          in_row = (uint32_t)c0b * 32 + g * 256 + (((P & 15) ^ (g & 3)) << 4);
        }
        lds_load16<kAuxNT>(rq, rl + h * 1024, in_row < rowq ? r * rowq + in_row : kOOB);
      }
    };
    uint4 xa[MT][4];
    float2 xd[MT];
    int2 xs[MT];
    auto load_act = [&](int c0b) {
#pragma unroll
      for (int m = 0; m < MT; m++) {
        if (MT == 1 || m < M) {
          const uint8_t* am = lds_act + (m * NCH + c0b / 128) * kActB;
          const uint8_t* ab = am + kb * 256;
          const int sw = kb & 3;
#pragma unroll
          for (int i = 0; i < 4; i++) xa[m][i] = *(const uint4*)(ab + (((4 * t + i) ^ sw) << 4));
          xd[m] = *(const float2*)(am + 4096 + (8 * kb + 2 * t) * 4);
          if constexpr (QT == UB_Q4_0) xs[m] = *(const int2*)(am + 4608 + (8 * kb + 2 * t) * 4);
        }
      }
    };
    // one chunk per row: the activation registers serve every unit (an LDS
    // read in the loop would also make the compiler drain the weight loads)
    if constexpr (NCH == 1) load_act(0);
    float acc[R * MT];
#pragma unroll
    for (int i = 0; i < R * MT; i++) acc[i] = 0.f;
    for (int c0b = 0; rg < nrg;) {
      const int row0 = (rg * W + wv) * R;
      const int nrows = rows_of(rg);
      int nrg_ = rg, nc0 = c0b + 128;
      if (nc0 >= nb) {
        nc0 = 0;
        nrg_ = rg + gridDim.x;
      }
      if (nrows > 0) {
        const int nrow0 = (nrg_ * W + wv) * R, nnrows = nrg_ < nrg ? rows_of(nrg_) : 0;
        if constexpr (NCH > 1) load_act(c0b);
#pragma unroll
        for (int r = 0; r < R; r++) {
          wait_vm_rows_pr<G::PR>(R - 1);
          const uint8_t* rl = row_lds(r);
          const uint32_t hv = *(const uint32_t*)(rl + G::QCB + kb * 16 + t * 4);
          uint4 q[4];
          if constexpr (QT == UB_Q4_0) {
            const int wsw = (kb >> 1) & 1;
            q[0] = *(const uint4*)(rl + kb * 128 + (((2 * t) ^ wsw) << 4));
            q[1] = *(const uint4*)(rl + kb * 128 + (((2 * t + 1) ^ wsw) << 4));
          } else {
            const uint8_t* qb = rl + kb * 256;
            const int sw = kb & 3;
#pragma unroll
            for (int i = 0; i < 4; i++) q[i] = *(const uint4*)(qb + (((4 * t + i) ^ sw) << 4));
          }
          __builtin_amdgcn_sched_barrier(0);
          __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the slice is read
          __builtin_amdgcn_sched_barrier(0);
          issue_row(nrow0, nnrows, nc0, r);
          const float dw0 = ub_f16_to_f32((uint16_t)(hv & 0xffff));
          const float dw1 = ub_f16_to_f32((uint16_t)(hv >> 16));
#pragma unroll
          for (int m = 0; m < MT; m++) {
            if (MT == 1 || m < M) {
              int s0, s1;
              if constexpr (QT == UB_Q4_0) {
                s0 = (dot_hi16(q[0], xa[m][1], 0) >> 4) + dot_lo(q[0], xa[m][0], 0) - 8 * xs[m].x;
                s1 = (dot_hi16(q[1], xa[m][3], 0) >> 4) + dot_lo(q[1], xa[m][2], 0) - 8 * xs[m].y;
              } else {
                s0 = dot_i8(q[1], xa[m][1], dot_i8(q[0], xa[m][0], 0));
                s1 = dot_i8(q[3], xa[m][3], dot_i8(q[2], xa[m][2], 0));
              }
              acc[r * MT + m] += (float)s0 * dw0 * xd[m].x;
              acc[r * MT + m] += (float)s1 * dw1 * xd[m].y;
            }
          }
        }
        if (nc0 == 0) {  // the row group is complete
          const float v = wave_reduce_scatter<R * MT>(acc, lane);
          constexpr int SH = 6 - ilog2<R * MT>();
          if ((lane & ((1 << SH) - 1)) == 0) {
            const int idx = lane >> SH;
            const int r = idx / MT, m = idx % MT;
            if (m < M && r < nrows) store_out<OT>(a.y, (size_t)m * N + row0 + r, v);
          }
#pragma unroll
          for (int i = 0; i < R * MT; i++) acc[i] = 0.f;
        }
      }
      rg = nrg_;
      c0b = nc0;
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): trailing out-of-range loads write the slices
    return;
  }

  for (bool first = true; rg < nrg; rg += gridDim.x, first = false) {
    const int row0 = (rg * W + wv) * R;
    const int nrows = rows_of(rg);
    float acc[R * MT];
#pragma unroll
    for (int i = 0; i < R * MT; i++) acc[i] = 0.f;
    for (int c0b = 0; c0b < nb; c0b += 128) {
      if (!first || c0b > 0) {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's reads of its slices have returned
        __builtin_amdgcn_sched_barrier(0);
        issue_rows(row0, nrows, c0b);
      }
      if (nrows == 0) continue;
      // activations of blocks 8 kb + 2t, + 1: units 4t .. 4t + 3 of group kb
      uint4 xa[MT][4];
      float2 xd[MT];
      int2 xs[MT];
#pragma unroll
      for (int m = 0; m < MT; m++) {
        if (MT == 1 || m < M) {
          const uint8_t* am = lds_act + (m * NCH + c0b / 128) * kActB;
          const uint8_t* ab = am + kb * 256;
          const int sw = kb & 3;
#pragma unroll
          for (int i = 0; i < 4; i++) xa[m][i] = *(const uint4*)(ab + (((4 * t + i) ^ sw) << 4));
          xd[m] = *(const float2*)(am + 4096 + (8 * kb + 2 * t) * 4);
          if constexpr (QT == UB_Q4_0) xs[m] = *(const int2*)(am + 4608 + (8 * kb + 2 * t) * 4);
        }
      }
#pragma unroll
      for (int r = 0; r < R; r++) {
        wait_vm_rows_pr<G::PR>(R - 1 - r);
        const uint8_t* rl = row_lds(r);
        const uint32_t hv = *(const uint32_t*)(rl + G::QCB + kb * 16 + t * 4);
        const float dw0 = ub_f16_to_f32((uint16_t)(hv & 0xffff));
        const float dw1 = ub_f16_to_f32((uint16_t)(hv >> 16));
        if constexpr (QT == UB_Q4_0) {
          const int wsw = (kb >> 1) & 1;
          const uint4 q0 = *(const uint4*)(rl + kb * 128 + (((2 * t) ^ wsw) << 4));
          const uint4 q1 = *(const uint4*)(rl + kb * 128 + (((2 * t + 1) ^ wsw) << 4));
#pragma unroll
          for (int m = 0; m < MT; m++) {
            if (MT == 1 || m < M) {
              const int s0 = (dot_hi16(q0, xa[m][1], 0) >> 4) + dot_lo(q0, xa[m][0], 0) - 8 * xs[m].x;
              const int s1 = (dot_hi16(q1, xa[m][3], 0) >> 4) + dot_lo(q1, xa[m][2], 0) - 8 * xs[m].y;
              acc[r * MT + m] += (float)s0 * dw0 * xd[m].x;
              acc[r * MT + m] += (float)s1 * dw1 * xd[m].y;
            }
          }
        } else {
          const uint8_t* qb = rl + kb * 256;
          const int sw = kb & 3;
          const uint4 q0 = *(const uint4*)(qb + (((4 * t) ^ sw) << 4));
          const uint4 q1 = *(const uint4*)(qb + (((4 * t + 1) ^ sw) << 4));
          const uint4 q2 = *(const uint4*)(qb + (((4 * t + 2) ^ sw) << 4));
          const uint4 q3 = *(const uint4*)(qb + (((4 * t + 3) ^ sw) << 4));
#pragma unroll
          for (int m = 0; m < MT; m++) {
            if (MT == 1 || m < M) {
              const int s0 = dot_i8(q1, xa[m][1], dot_i8(q0, xa[m][0], 0));
              const int s1 = dot_i8(q3, xa[m][3], dot_i8(q2, xa[m][2], 0));
              acc[r * MT + m] += (float)s0 * dw0 * xd[m].x;
              acc[r * MT + m] += (float)s1 * dw1 * xd[m].y;
            }
          }
        }
      }
    }
    if (nrows == 0) continue;
    const float v = wave_reduce_scatter<R * MT>(acc, lane);
    constexpr int SH = 6 - ilog2<R * MT>();
    if ((lane & ((1 << SH) - 1)) == 0) {
      const int idx = lane >> SH;
      const int r = idx / MT, m = idx % MT;
      if (m < M && r < nrows) store_out<OT>(a.y, (size_t)m * N + row0 + r, v);
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): loads of rows past N still write the slices
}


template <int QT, int MT, int R, int U, int OT>
void launch_t(const GemvArgs& a, hipStream_t s) {
  k_gemv<QT, MT, R, U, OT><<<ub_cdiv(a.N, kWaves * R), 256, 0, s>>>(a);
}

// One-launch QMatMul for Q4_0 / Q8_0 with 1-2 tokens (k_gemv quantizing the
// activations itself): 4 waves x R rows per workgroup, R = 4 for Q4_0 (fewer
// workgroups repeating the quantization) and 2 for Q8_0 (measured on MI355X:
// Q4_0 4096 x 4096 6.25 us, Q8_0 4096 x 4096 7.1 us against 6.4 / 8.7 us for
// quantize + GEMV launches); gemv_rows overrides with 1, 2 or 4, and
// gemv_iters = 1 takes one block-iteration per pass instead of two.
template <int QT, int MT, int OT, int XQ>
void launch_fused_q80(const GemvArgs& a, hipStream_t s) {
  const int env_r = ub_tune(UB_TUNE_GEMV_ROWS);
  const int r = env_r ? env_r : (QT == UB_Q4_0 ? 4 : 2);
  if (ub_tune(UB_TUNE_GEMV_ITERS) == 1) {
    if (r == 1) k_gemv<QT, MT, 1, 1, OT, XQ><<<ub_cdiv(a.N, kWaves), 256, 0, s>>>(a);
    else if (r >= 4) k_gemv<QT, MT, 4, 1, OT, XQ><<<ub_cdiv(a.N, kWaves * 4), 256, 0, s>>>(a);
    else k_gemv<QT, MT, 2, 1, OT, XQ><<<ub_cdiv(a.N, kWaves * 2), 256, 0, s>>>(a);
    return;
  }
  // two block-iterations per pass: at K = 4096 every weight load of the row
  // is in flight while the activations are quantized
  if (r == 1) k_gemv<QT, MT, 1, 2, OT, XQ><<<ub_cdiv(a.N, kWaves), 256, 0, s>>>(a);
  else if (r >= 4) k_gemv<QT, MT, 4, 2, OT, XQ><<<ub_cdiv(a.N, kWaves * 4), 256, 0, s>>>(a);
  else k_gemv<QT, MT, 2, 2, OT, XQ><<<ub_cdiv(a.N, kWaves * 2), 256, 0, s>>>(a);
}
template <int QT, int OT, int XQ>
void launch_fused_q80_m(const GemvArgs& a, hipStream_t s) {
  if (a.M == 1) launch_fused_q80<QT, 1, OT, XQ>(a, s);
  else launch_fused_q80<QT, 2, OT, XQ>(a, s);
}
// LDS-staged form (k_gemv_q80_pq): K a multiple of 256 up to 16384; grid
// min(row groups, resident workgroups); W wavefronts x R rows per group
// (gemv_lds_waves / gemv_lds_rows override the default 4 x 2).
template <int QT, int W, int MT, int R, int OT, int XQ, int NCH, bool ROLL>
void launch_q80_pq_t(const GemvArgs& a, hipStream_t s) {
  static int resident = 0;
  if (resident == 0) {
    int per_cu = 0, dev = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, k_gemv_q80_pq<QT, W, MT, R, OT, XQ, NCH, ROLL>, 64 * W, 0) != hipSuccess ||
        per_cu < 1)
      per_cu = 1;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus < 1)
      cus = 256;
    resident = per_cu * cus;
  }
  const int nrg = ub_cdiv(a.N, W * R);
  k_gemv_q80_pq<QT, W, MT, R, OT, XQ, NCH, ROLL><<<nrg < resident ? nrg : resident, 64 * W, 0, s>>>(a);
}
template <int QT, int W, int MT, int R, int OT, int XQ, bool ROLL>
void launch_q80_pq_r(const GemvArgs& a, hipStream_t s) {
  const int nch = ub_cdiv(a.K, 4096);
  if (nch <= 1) launch_q80_pq_t<QT, W, MT, R, OT, XQ, 1, ROLL>(a, s);
  else if (nch <= 2) launch_q80_pq_t<QT, W, MT, R, OT, XQ, 2, ROLL>(a, s);
  else launch_q80_pq_t<QT, W, MT, R, OT, XQ, 4, ROLL>(a, s);
}
// The rolling prefetch (see k_gemv_q80_pq) from 2 tokens where a workgroup
// walks several units: the wide layer (N >= 16384, more row groups than
// resident workgroups) and K > 4096 (several chunks per row).  Measured on
// MI355X (Q8_0, us, rolling / not): 4096 x 28672 2-4 tokens 20.1 / 20.7,
// 21.3 / 21.7, 22.1 / 22.8; 14336 x 4096 3-4 tokens 18.4 / 19.0, 20.5 /
// 21.2; but 4096 x 6144 at 2 tokens 7.8 / 6.7 and one token 1-3% slower
// everywhere.  gemv_persist = 2 / 3 forces it off / on.
template <int QT, int W, int MT, int R, int OT, int XQ>
void launch_q80_pq_n(const GemvArgs& a, hipStream_t s) {
  const int pmode = ub_tune(UB_TUNE_GEMV_PERSIST);
  if (pmode == 3 || (pmode != 2 && MT > 1 && (a.N >= 16384 || a.K > 4096)))
    launch_q80_pq_r<QT, W, MT, R, OT, XQ, true>(a, s);
  else launch_q80_pq_r<QT, W, MT, R, OT, XQ, false>(a, s);
}
// Default shape 8 wavefronts x 2 rows (Q4_0) or x 1 row (Q8_0), from a sweep
// of the Llama-3-8B decode shapes on MI355X.
template <int QT, int MT, int OT, int XQ>
void launch_q80_pq_m(const GemvArgs& a, hipStream_t s) {
  int r = ub_tune(UB_TUNE_GEMV_LDS_ROWS), w = ub_tune(UB_TUNE_GEMV_LDS_WAVES);
  if (r <= 0 && w <= 0) {
    w = 8;
    r = QT == UB_Q8_0 ? 1 : 2;
  }
  if (w == 8) {
    if (r == 1) return launch_q80_pq_n<QT, 8, MT, 1, OT, XQ>(a, s);
    return launch_q80_pq_n<QT, 8, MT, 2, OT, XQ>(a, s);
  }
  if (r == 1) return launch_q80_pq_n<QT, 4, MT, 1, OT, XQ>(a, s);
  if (r >= 4) return launch_q80_pq_n<QT, 4, MT, 4, OT, XQ>(a, s);
  launch_q80_pq_n<QT, 4, MT, 2, OT, XQ>(a, s);
}
bool q80_lds_ok(const GemvArgs& a) {
  return ub_tune(UB_TUNE_GEMV_Q80_LDS) >= 0 && a.K % 256 == 0 && a.K <= 16384;
}
template <int QT, int OT, int XQ>
void launch_q80_pq(const GemvArgs& a, hipStream_t s) {
  if (a.M == 1) launch_q80_pq_m<QT, 1, OT, XQ>(a, s);
  else if (a.M == 2) launch_q80_pq_m<QT, 2, OT, XQ>(a, s);
  else launch_q80_pq_m<QT, 4, OT, XQ>(a, s);
}

template <int QT>
void launch_fused_q80_t(int x_dt, int y_dt, const GemvArgs& a, hipStream_t s) {
  if (q80_lds_ok(a)) {
    if (y_dt == UB_F32) {
      if (x_dt == UB_F32) launch_q80_pq<QT, UB_F32, UB_F32>(a, s);
      else launch_q80_pq<QT, UB_F32, UB_BF16>(a, s);
    } else {
      if (x_dt == UB_F32) launch_q80_pq<QT, UB_BF16, UB_F32>(a, s);
      else launch_q80_pq<QT, UB_BF16, UB_BF16>(a, s);
    }
    return;
  }
  if (y_dt == UB_F32) {
    if (x_dt == UB_F32) launch_fused_q80_m<QT, UB_F32, UB_F32>(a, s);
    else launch_fused_q80_m<QT, UB_F32, UB_BF16>(a, s);
  } else {
    if (x_dt == UB_F32) launch_fused_q80_m<QT, UB_BF16, UB_F32>(a, s);
    else launch_fused_q80_m<QT, UB_BF16, UB_BF16>(a, s);
  }
}

template <int MT, int R, int OT, int XQ>
void launch_lds(int w, const GemvArgs& a, hipStream_t s) {
  if constexpr (R * 16 * 2304 + MT * 5120 <= 160 * 1024) {  // 16 wavefronts: LDS permitting
    if (w >= 16) return k_gemv_q4k_lds<16, MT, R, OT, XQ><<<ub_cdiv(a.N, 16 * R), 1024, 0, s>>>(a);
  }
  if (w >= 8) k_gemv_q4k_lds<8, MT, R, OT, XQ><<<ub_cdiv(a.N, 8 * R), 512, 0, s>>>(a);
  else k_gemv_q4k_lds<4, MT, R, OT, XQ><<<ub_cdiv(a.N, 4 * R), 256, 0, s>>>(a);
}

// Shape of the LDS-staged Q4_K kernel, from a sweep of the Llama-3-8B decode
// shapes on MI355X.  With workspace activations (XQ < 0): four wavefronts per
// workgroup, R = 2 rows per wavefront for the wide layers (N >= 16384), else
// 1; with 3-4 tokens (MT = 4) R = 4 / 2 (the register path it replaces there
// measured 25-40% slower).  When the kernel also quantizes (XQ >= 0) every workgroup repeats that
// work, so the workgroups cover more rows: 4 waves x 4 rows for the wide
// layers, 8 waves x 2 rows for the rest.
// The gemv_lds_rows (R; < 0 switches the LDS path off) and gemv_lds_waves
// knobs override the choice.
bool lds_enabled() { return ub_tune(UB_TUNE_GEMV_LDS_ROWS) >= 0; }
// Persistent form: as many workgroups as stay resident (occupancy x CUs,
// looked up once per kernel), at most one per row group and 5 per CU; with
// the rolling prefetch 1-3 workgroups per CU, so that each walks ~3 or more
// row groups.  Measured on MI355X, Q4_K K = 4096 (us): N = 28672 at grids
// of 768 / 1024 / 1280 / 1536, one token 12.1 / 12.0 / 11.6 / 12.3-12.8,
// two tokens (rolling) 12.8 / 13.5 / 14.4 / 15.2; N = 6144 (768 row
// groups), 4 tokens rolling at 256 / 384 / 512 / 768 workgroups 8.5 / 10.0
// / 9.2 / 10.6; grids of fractional workgroups per CU measured 5-15%
// slower.
int cu_count() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, v = 0;
    cus = hipGetDevice(&dev) == hipSuccess &&
                  hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
                  v > 0
              ? v
              : 256;
  }
  return cus;
}
template <int W, int MT, int R, int OT, int XQ, int NCH, bool ROLL>
int pq_resident() {
  static int resident = 0;
  if (resident == 0) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_gemv_q4k_pq<W, MT, R, OT, XQ, NCH, ROLL>,
                                                     64 * W, 0) != hipSuccess || per_cu < 1)
      per_cu = 1;
    resident = std::min(per_cu, ROLL ? 3 : 5) * cu_count();
  }
  return resident;
}
template <int W, int MT, int R, int OT, int XQ, int NCH, bool ROLL>
void launch_pq_t(const GemvArgs& a, hipStream_t s) {
  const int resident = pq_resident<W, MT, R, OT, XQ, NCH, ROLL>();
  const int nrg = ub_cdiv(a.N, W * R);
  int grid = std::min(nrg, resident);
  if (ROLL) {  // whole workgroups per CU, each walking about 3 or more row groups
    const int cus = cu_count();
    grid = std::min({nrg, resident, std::max(1, std::min(3, nrg / (3 * cus))) * cus});
  }
  k_gemv_q4k_pq<W, MT, R, OT, XQ, NCH, ROLL><<<grid, 64 * W, 0, s>>>(a);
}
template <int W, int MT, int R, int OT, int XQ, bool ROLL>
bool launch_pq_nch(const GemvArgs& a, hipStream_t s) {
  const int nbr = a.K / 256;
  if (nbr <= kQ4kCB) launch_pq_t<W, MT, R, OT, XQ, 1, ROLL>(a, s);
  else if (nbr <= 2 * kQ4kCB) launch_pq_t<W, MT, R, OT, XQ, 2, ROLL>(a, s);
  else if (nbr <= 4 * kQ4kCB) launch_pq_t<W, MT, R, OT, XQ, 4, ROLL>(a, s);
  else return false;
  return true;
}
// Rolling prefetch from 2 tokens; at one token the form that issues a row
// group's loads after the previous group's math.  Measured on MI355X, Q4_K
// 4096 x 28672 (us, rolling / not): 1 token 12.7-13.0 / 11.4-11.6, 2 tokens
// 13.1 / 14.7, 3 tokens 15.4 / 18.7, 4 tokens 17.9 / 20.6.  gemv_persist = 2
// forces the non-rolling form, 3 the rolling one.
template <int W, int MT, int R, int OT, int XQ>
bool launch_pq_w(const GemvArgs& a, hipStream_t s) {
  const int pmode = ub_tune(UB_TUNE_GEMV_PERSIST);
  const bool roll = pmode == 3 || (pmode != 2 && MT > 1);
  return roll ? launch_pq_nch<W, MT, R, OT, XQ, true>(a, s)
              : launch_pq_nch<W, MT, R, OT, XQ, false>(a, s);
}

template <int MT, int OT, int XQ>
void launch_lds_r(const GemvArgs& a, hipStream_t s) {
  const int env_r = ub_tune(UB_TUNE_GEMV_LDS_ROWS), env_w = ub_tune(UB_TUNE_GEMV_LDS_WAVES);
  const bool wide = a.N >= 16384;
  int r = XQ < 0 ? (MT > 2 ? (wide ? 4 : 2) : (wide ? 2 : 1)) : (wide ? 4 : 2);
  int w = XQ >= 0 && !wide ? 8 : 4;
  if (env_r > 0) r = env_r;
  if (env_w > 0) w = env_w;
  if constexpr (XQ >= 0) {
    // The persistent grid (4 wavefronts x 2 rows, x quantized once per
    // workgroup) when the rows outnumber what stays resident and one chunk
    // holds the row (K <= 4096); measured on MI355X: Q4_K 4096 x 28672 at
    // 1 token 11.5 us against 12.5 us for the one-shot grid, 2 tokens 14.2
    // against 16.2 us; the narrow layers and K = 14336 stay faster one-shot.
    // Switch-over (measured on MI355X, K = 4096, us one-shot / persistent):
    // one token from N = 16384 (11008: 6.5 / 7.2, 16384: 8.6 / 8.0), 2-4
    // tokens (rolling) from N = 6144 (4096 x 4 tokens 6.9 / 8.2; 6144 x 2 /
    // 3 / 4 tokens 6.6 / 6.5, 10.1 / 7.5, 11.9 / 8.5; 11008 x 4 17.5 /
    // 11.4).
    const int pmode = ub_tune(UB_TUNE_GEMV_PERSIST);
    bool persist = pmode > 0;
    if (pmode == 0 && a.K <= 256 * kQ4kCB && env_r <= 0 && env_w <= 0)
      persist = MT == 1 ? a.N >= 16384 : a.N >= 6144;
    if (persist) {
      if (env_r >= 4 ? launch_pq_w<4, MT, 4, OT, XQ>(a, s) : launch_pq_w<4, MT, 2, OT, XQ>(a, s))
        return;
    }
  }
  if (r >= 4) return launch_lds<MT, 4, OT, XQ>(w, a, s);
  if (r == 2) return launch_lds<MT, 2, OT, XQ>(w, a, s);
  launch_lds<MT, 1, OT, XQ>(w, a, s);
}

// Rows per wavefront (R) and block-iterations per pass (U), from a sweep of
// the Llama-3-8B decode shapes on MI355X: R = 2 keeps ~8 KiB in flight per
// wavefront without cutting occupancy; R = 4 only pays for the widest Q4_K
// layers at M = 1; U = 2 only for Q4_K with >= 2 iterations (K >= 8192).
// The gemv_rows / gemv_iters knobs override the choice.
template <int QT, int MT, int OT>
void launch_ru(const GemvArgs& a, hipStream_t s) {
  using G = Geo<QT>;
  const int env_r = ub_tune(UB_TUNE_GEMV_ROWS), env_u = ub_tune(UB_TUNE_GEMV_ITERS);
  const int iters = (a.K / G::BK + G::BPI - 1) / G::BPI;
  int r = 2;
  if (QT == UB_Q4_K && MT == 1 && a.N >= 16384) r = 4;
  if (QT == UB_Q8_0 && a.N < 8192 && MT == 1) r = 1;
  if (env_r) r = env_r;
  if constexpr (QT == UB_Q4_K && MT <= 4) {
    if (lds_enabled()) return launch_lds_r<MT, OT, -1>(a, s);
  }
  const bool u2 = env_u ? env_u >= 2 : (QT == UB_Q4_K && iters >= 2);
  if (u2) {
    if (r == 4 && MT <= 4) return launch_t<QT, MT, 4, 2, OT>(a, s);
    if (r >= 2) return launch_t<QT, MT, 2, 2, OT>(a, s);
    return launch_t<QT, MT, 1, 2, OT>(a, s);
  }
  if (r == 4 && MT <= 4) return launch_t<QT, MT, 4, 1, OT>(a, s);
  if (r >= 2) return launch_t<QT, MT, 2, 1, OT>(a, s);
  launch_t<QT, MT, 1, 1, OT>(a, s);
}

// ------------------------------------------- multi-token GEMV on int8 MFMA
// The per-token VALU dot products of k_gemv grow with M; here the integer
// block dots come from
// v_mfma_i32_16x16x32_i8 instead: one MFMA takes a 16-row x 32-k tile of
// weights (one Q8_0 block / one Q4_K sub-block, nibbles widened to int8) and
// the same 32 k of all 16 token slots (tokens >= M read zero), and returns
// the 16 x 16 exact int32 block dots.  Lane l supplies row / token l % 16 at
// k = 8 (l / 16) .. +7 and receives rows 4 (l / 16) + i of token l % 16.  The
// VALU work left is the per-block scaling of each output (for Q4_K the
// min term sum_j dmin*m_j * d_a*s_j is itself a small f32 MFMA per block).
// The ring GEMV below (k_gemv_mm) takes 5..16 tokens when K is a multiple
// of 1024; otherwise this kernel does for Q4_K, while Q8_0 keeps the register
// path (measured as fast up to 16 tokens) unless the gemv_mfma_m knob asks.
//
// A workgroup of 8 wavefronts owns 16 rows; the wavefronts split K into
// 512-element chunks (chunk c goes to wave c % 8), each streaming its rows'
// chunk into its own LDS slice with direct-to-LDS loads, and the 8 partial
// results are summed through LDS at the end (a fixed order: deterministic).
// The code slice of each row is XOR-swizzled in 16-byte units by the row
// index, so the 16 rows a fragment read touches fall in distinct banks.
// Before the MFMAs each wave turns its chunk's block headers into f32 scale
// tables in LDS (d, or d*sc and dmin*m per Q4_K sub-block), laid out so a
// lane reads the scales of its four output rows with one 16-byte read.
constexpr int kMKC = 512;  // elements per chunk

template <int QT, int OT, int kMW>
__global__ void __launch_bounds__(64 * kMW) k_gemv_mfma(GemvArgs a) {
  static_assert(QT == UB_Q8_0 || QT == UB_Q4_K, "MFMA GEMV: Q8_0 or Q4_K");
  constexpr int CODEB = QT == UB_Q8_0 ? 512 : 256;  // code bytes per row and chunk
  constexpr int CH = CODEB / 16;                     // 16-byte units per row and chunk
  constexpr int HDRB = 32;                           // header bytes per row and chunk
  constexpr int NTAB = QT == UB_Q4_K ? 2 : 1;        // scale tables
  constexpr int NDA = QT == UB_Q8_0 ? 16 : 2;        // activation scales per chunk
  __shared__ __attribute__((aligned(16))) uint8_t lc[kMW * 16 * CODEB];
  __shared__ __attribute__((aligned(16))) uint8_t lh[kMW * 16 * HDRB];
  __shared__ __attribute__((aligned(16))) float lsc[kMW * NTAB * 256];
  __shared__ __attribute__((aligned(16))) float lred[kMW * 256];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tok = lane & 15, h = lane >> 4;
  const int row0 = blockIdx.x * 16;
  const int N = a.N, K = a.K, M = a.M;
  const int nrows = min(16, N - row0);
  const uint32_t rowcb = QT == UB_Q8_0 ? K : K / 2;  // code bytes per row
  const uint32_t rowhb = K / 16;                     // header bytes per row
  const __amdgpu_buffer_rsrc_t rq =
      rsrc_u(a.w + a.nbw * (QT == UB_Q8_0 ? 2 : 16) + (size_t)row0 * rowcb, nrows * rowcb);
  const __amdgpu_buffer_rsrc_t rh = rsrc_u(a.w + (size_t)row0 * rowhb, nrows * rowhb);
  const __amdgpu_buffer_rsrc_t raq = rsrc_u(a.qa, (uint32_t)(M * K));
  const int nda_row = QT == UB_Q8_0 ? K / 32 : K / 256;
  const __amdgpu_buffer_rsrc_t rad = rsrc_u(a.da, (uint32_t)(M * nda_row * 4));
  const __amdgpu_buffer_rsrc_t ras = rsrc_u(a.sa, (uint32_t)(M * (K / 32) * 4));
  uint8_t* wc = lc + wv * 16 * CODEB;
  uint8_t* wh = lh + wv * 16 * HDRB;
  float* ws = lsc + wv * NTAB * 256;

  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  const int nch = (K + kMKC - 1) / kMKC;
  for (int c = wv; c < nch; c += kMW) {
    // activations: the B fragment of each 32-k block, and the scales
    uint2 bq[16];
#pragma unroll
    for (int sb = 0; sb < 16; sb++) {
      const uint32_t e = (uint32_t)c * kMKC + 32 * sb + 8 * h;
      bq[sb] = bload8(raq, tok < M && e < (uint32_t)K ? (uint32_t)tok * K + e : kOOB);
    }
    float dav[NDA];
#pragma unroll
    for (int j = 0; j < NDA; j++) {
      const uint32_t bi = (uint32_t)c * NDA + j;  // block index in the token's row
      dav[j] = __uint_as_float(
          bload4(rad, tok < M && bi < (uint32_t)nda_row ? (tok * nda_row + bi) * 4 : kOOB));
    }
    // Q4_K: the 32-element code sums this lane feeds to the min-term MFMA:
    // token tok, sub-blocks 8b + 4q + h of the chunk (b, q in {0, 1})
    int sav[QT == UB_Q4_K ? 4 : 1];
    if constexpr (QT == UB_Q4_K) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t si = (uint32_t)c * 16 + 4 * j + h;
        sav[j] = (int)bload4(ras, tok < M && si < (uint32_t)(K / 32) ? (tok * (K / 32) + si) * 4 : kOOB);
      }
    }
    // weights -> LDS: codes (16-byte unit u of row r lands at unit u ^ r),
    // then the block headers
#pragma unroll
    for (int i = 0; i < 16 * CODEB / 1024; i++) {
      const int p = i * 1024 + lane * 16;
      const int r = p / CODEB, u = (p % CODEB) / 16;
      const uint32_t in_row = (uint32_t)c * CODEB + ((u ^ (r & (CH - 1))) * 16);
      lds_load16<kAuxNT>(rq, wc + i * 1024, in_row < rowcb ? r * rowcb + in_row : kOOB);
    }
    // Q4_K headers -> LDS.  (Q8_0 header rows are K/16 bytes, only 2-byte
    // aligned, and direct-to-LDS loads need dword-aligned addresses: this
    // lane's four scales are loaded into registers instead.)
    uint32_t hq[QT == UB_Q8_0 ? 4 : 1];
    if constexpr (QT == UB_Q8_0) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t in_row = (uint32_t)c * HDRB + 2 * (4 * h + j);
        hq[j] = bload2(rh, in_row < rowhb ? (lane & 15) * rowhb + in_row : kOOB);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16 * HDRB / 256; i++) {
        const int p = i * 256 + lane * 4;
        const int r = p / HDRB;
        const uint32_t in_row = (uint32_t)c * HDRB + p % HDRB;
        lds_load4<kAuxNT>(rh, wh + i * 256, in_row < rowhb ? r * rowhb + in_row : kOOB);
      }
    }
    wait_vm();
    // scale tables [sub-block][row]
    {
      const int r = lane & 15;
      if constexpr (QT == UB_Q8_0) {
#pragma unroll
        for (int j = 0; j < 4; j++) ws[(4 * h + j) * 16 + r] = ub_f16_to_f32((uint16_t)hq[j]);
      } else {
        const int b = h & 1, q = h >> 1;  // block of the chunk; sub-blocks 4q..4q+3
        const uint4 hd = *(const uint4*)(wh + r * HDRB + 16 * b);
        const float d = ub_f16_to_f32((uint16_t)(hd.x & 0xffff));
        const float dmin = ub_f16_to_f32((uint16_t)(hd.x >> 16));
        auto byte = [&](int i) -> int {  // scale byte i (0..11); i is lane-dependent
          const uint32_t w = i < 4 ? hd.y : (i < 8 ? hd.z : hd.w);
          return (int)((w >> (8 * (i & 3))) & 0xff);
        };
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int js = 4 * q + j;  // get_scale_min_k4 (quant.cpp:356-363)
          int scv, mv;
          if (js < 4) {
            scv = byte(js) & 63;
            mv = byte(js + 4) & 63;
          } else {
            scv = (byte(js + 4) & 0xF) | ((byte(js - 4) >> 6) << 4);
            mv = (byte(js + 4) >> 4) | ((byte(js) >> 6) << 4);
          }
          ws[(8 * b + js) * 16 + r] = d * (float)scv;
          ws[256 + (8 * b + js) * 16 + r] = dmin * (float)mv;
        }
      }
    }
    // block dots on MFMA, scaled per block
    typedef int i32x4 __attribute__((ext_vector_type(4)));
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const i32x4 izero = {0, 0, 0, 0};
    const int r = lane & 15;
    if constexpr (QT == UB_Q8_0) {
#pragma unroll
      for (int sb = 0; sb < 16; sb++) {
        const int u = 2 * sb + (h >> 1);
        const uint2 av = *(const uint2*)(wc + r * CODEB + ((u ^ (r & (CH - 1))) * 16) + 8 * (h & 1));
        const i32x4 I = __builtin_amdgcn_mfma_i32_16x16x32_i8(
            (long)(((uint64_t)av.y << 32) | av.x), (long)(((uint64_t)bq[sb].y << 32) | bq[sb].x),
            izero, 0, 0, 0);
        const float4 dsc = *(const float4*)(ws + sb * 16 + 4 * h);
        const float f = dav[sb];
        acc[0] += (dsc.x * f) * (float)I[0];
        acc[1] += (dsc.y * f) * (float)I[1];
        acc[2] += (dsc.z * f) * (float)I[2];
        acc[3] += (dsc.w * f) * (float)I[3];
      }
    } else {
#pragma unroll
      for (int b = 0; b < 2; b++) {
        // sum_j d*sc[n][j] * dot[n][tok][j] over the block's 8 sub-blocks
        float T[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const int sb = 8 * b + j;
          const int u = 8 * b + 2 * (j >> 1) + (h >> 1);
          const uint2 raw =
              *(const uint2*)(wc + r * CODEB + ((u ^ (r & (CH - 1))) * 16) + 8 * (h & 1));
          const int sh = 4 * (j & 1);
          const uint2 av = make_uint2((raw.x >> sh) & 0x0F0F0F0Fu, (raw.y >> sh) & 0x0F0F0F0Fu);
          const i32x4 I = __builtin_amdgcn_mfma_i32_16x16x32_i8(
              (long)(((uint64_t)av.y << 32) | av.x), (long)(((uint64_t)bq[sb].y << 32) | bq[sb].x),
              izero, 0, 0, 0);
          const float4 dsc = *(const float4*)(ws + sb * 16 + 4 * h);
          T[0] += dsc.x * (float)I[0];
          T[1] += dsc.y * (float)I[1];
          T[2] += dsc.z * (float)I[2];
          T[3] += dsc.w * (float)I[3];
        }
        // min term sum_j dmin*m[n][j] * (d_a * sum_a)[tok][j] as two f32 MFMAs
        // (k = 4 sub-blocks each): lane supplies row / token l % 16, k = l / 16
        f32x4 mn = {0.f, 0.f, 0.f, 0.f};
        const float f = dav[b];
#pragma unroll
        for (int q = 0; q < 2; q++) {
          const float am = ws[256 + (8 * b + 4 * q + h) * 16 + r];
          mn = __builtin_amdgcn_mfma_f32_16x16x4f32(am, f * (float)sav[2 * b + q], mn, 0, 0, 0);
        }
        acc[0] += f * T[0] - mn[0];
        acc[1] += f * T[1] - mn[1];
        acc[2] += f * T[2] - mn[2];
        acc[3] += f * T[3] - mn[3];
      }
    }
  }
  // sum the 8 wavefronts' partials: lred[w][row][token]
#pragma unroll
  for (int i = 0; i < 4; i++) lred[wv * 256 + (4 * h + i) * 16 + tok] = acc[i];
  __syncthreads();
  if (threadIdx.x < 256) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kMW; w++) v += lred[w * 256 + threadIdx.x];
    const int rr = threadIdx.x >> 4, t = threadIdx.x & 15;
    if (t < M && rr < nrows) store_out<OT>(a.y, (size_t)t * N + row0 + rr, v);
  }
}

// ---------------------------------- multi-token GEMV: direct-to-LDS ring
// Decode batches of 3..16 tokens.  The whole GEMV is HBM-bound on the weight
// (one pass over [N, K] packed blocks), so the kernel is built around
// streaming it: a workgroup owns RT = 16 RWV consecutive rows and walks K in
// steps of KG SB 256 elements through a D-stage ring of LDS buffers filled by
// direct-to-LDS loads (weight codes; activations: the Q8_K / Q8_0 workspace
// codes, sums and scales of all 16 token slots).  The tile's block headers
// are loaded once, at the start, as one contiguous run per row.  The
// activations of a step are loaded once per workgroup and shared by its RWV
// row wavefronts (RT rows per activation byte instead of the 16 of k_gemv_mfma);
// the KG wavefront groups take disjoint SB-super-block slices of each step and
// are summed through LDS at the end in a fixed order.
//
// Each wavefront computes its 16 rows x 16 tokens with
// v_mfma_i32_16x16x32_i8: one MFMA per 32-element block (Q8_0 / Q4_0 block,
// Q4_K sub-block; 4-bit codes are widened to bytes on the way from LDS, Q4_0's
// as the signed q - 8), exact int32 block dots.  Q8_0 / Q4_0: acc += (d_w
// d_a) * dot.  Q4_K: the sub-block
// scales are applied in integer (sum_j sc_j dot_j, < 2^25) and the result
// scaled once per super-block by d_w d_a; the min term
// sum_j dmin m_j * d_a s_j is accumulated by v_mfma_f32_16x16x4f32.  LDS
// rows are padded by one 16-byte unit so the 16 rows (tokens) of a fragment
// read fall in distinct banks, and every read is a per-step base plus a
// constant offset.
//
// Load bookkeeping: a wavefront issues PW load instructions per step, or PW -
// 1 when the step's TI instructions leave its last slot empty (such a slot
// issues nothing: an out-of-range load would still write zeros into LDS), so
// "stage s has landed" is one of two immediate vmcnts; one s_barrier per step then
// publishes the stage to the workgroup and frees the stage read in the
// previous step for the next loads.  Steps past the end of K issue the same
// loads with out-of-range offsets (zero, no memory traffic).
// Requires K % 1024 == 0 (every variant's step, up to 4 super-blocks, divides
// the row) and weight / workspace buffers below 2 GiB (32-bit offsets with an
// out-of-range marker).
template <int QT, int RWV, int KG, int SB>
struct MmCfg {
  static constexpr int NW = RWV * KG;                  // wavefronts
  static constexpr int RT = 16 * RWV;                  // rows per workgroup
  static constexpr int CB = QT == UB_Q8_0 ? 256 : 128; // code bytes per row and 256 elements
  static constexpr int CU = SB * CB / 16;              // code units (16 B) per row and group
  static constexpr int pad(int u) { return (u + 63) / 64 * 64; }
  // regions of a stage, in 16-byte units; one load instruction fills 64
  // units (1 KiB), except the Q4_K activation scales: dword loads, 16 units.
  // Code rows and activation token rows carry one pad unit each.
  static constexpr int CUP = CU + 1;                   // units per code row in LDS
  static constexpr int AUP = SB * 16 + 1;              // units per activation row in LDS
  static constexpr int WC = KG * RT * CUP;             // weight codes
  static constexpr int AC = KG * 16 * AUP;             // activation codes
  static constexpr int AS = QT == UB_Q4_K ? KG * 16 * 2 * SB : 0;  // Q8_K sub-block sums
  static constexpr int NDW = KG * 16 * SB;                          // Q4_K: Q8_K scales (dwords)
  static constexpr int IAD = QT == UB_Q4_K ? (NDW + 63) / 64 : pad(KG * 16 * 2 * SB) / 64;
  static constexpr int AD = QT == UB_Q4_K ? 16 * IAD : 64 * IAD;    // activation scales
  static constexpr int oWC = 0, oAC = oWC + pad(WC), oAS = oAC + pad(AC), oAD = oAS + pad(AS),
                       SU = oAD + AD;  // units per stage
  static constexpr int IWC = pad(WC) / 64, IAC = pad(AC) / 64, IAS = pad(AS) / 64;
  static constexpr int TI = IWC + IAC + IAS + IAD;  // load instructions per step
  static constexpr int PW = (TI + NW - 1) / NW;           // per wavefront (at most)
};

template <int QT, int OT, int RWV, int KG, int SB, int D, int HK>
__global__ void __launch_bounds__(64 * RWV * KG) k_gemv_mm(GemvArgs a) {
  using C = MmCfg<QT, RWV, KG, SB>;
  constexpr int NW = C::NW, RT = C::RT, PW = C::PW;
  static_assert(D >= 2 && D * PW <= 63, "ring depth / vmcnt range");
  __shared__ __attribute__((aligned(16))) uint8_t ring[D * C::SU * 16];
  // header units rounded up to whole 64-unit load instructions: the last
  // instruction's out-of-range lanes still write (zeros) into LDS
  constexpr int HU = (RT * (HK + 1) + 63) / 64 * 64;
  __shared__ __attribute__((aligned(16))) uint8_t hdr[HU * 16];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rw = wv % RWV, gw = wv / RWV;
  const int r = lane & 15, h = lane >> 4;
  const int row0 = blockIdx.x * RT;
  const int N = a.N, K = a.K, M = a.M;
  const int nbr = K / 256;
  const int nsteps = nbr / (KG * SB);
  const uint32_t hdrb = QT == UB_Q4_K ? 16u : 2u;
  const uint32_t codes_at = (uint32_t)(a.nbw * hdrb);
  const uint32_t wbytes = codes_at + (uint32_t)((size_t)N * K / (QT == UB_Q8_0 ? 1 : 2));
  const ub_u32x4 dw_ = ub_desc(a.w, wbytes);
  const uint8_t* qa = (const uint8_t*)a.qa;
  const uint32_t off_d = (uint32_t)((const uint8_t*)a.da - qa);
  const uint32_t off_s = (uint32_t)((const uint8_t*)a.sa - qa);
  const uint32_t abytes =
      QT == UB_Q4_K ? off_s + (uint32_t)(M * (K / 32) * 4) : off_d + (uint32_t)(M * (K / 32) * 4);
  const ub_u32x4 da_ = ub_desc(qa, abytes);
  const uint32_t ring0 = ub_lds_addr(ring);

  // Load instruction `ins` (0..TI-1) of a step: region boundaries, the
  // lane's byte offset at step 0 (kOOB where the lane loads nothing) and the
  // per-step advance, which is the same for every lane of the instruction.
  constexpr int B1 = C::IWC, B3 = B1 + C::IAC, B4 = B3 + C::IAS;
  auto ins_inc = [&](int ins) -> uint32_t {
    constexpr uint32_t S = KG * SB;  // super-blocks per step
    if (ins < B1) return S * C::CB;
    if (ins < B3) return S * 256;
    if (ins < B4) return S * 32;
    return QT == UB_Q4_K ? S * 4 : S * 32;
  };
  auto ins_lds = [&](int ins) -> uint32_t {  // byte offset in a stage
    if (ins < B1) return (C::oWC + 64 * ins) * 16;
    if (ins < B3) return (C::oAC + 64 * (ins - B1)) * 16;
    if (ins < B4) return (C::oAS + 64 * (ins - B3)) * 16;
    return (C::oAD + (QT == UB_Q4_K ? 16 : 64) * (ins - B4)) * 16;
  };
  auto base_off = [&](int ins) -> uint32_t {
    const int P = (ins < B1 ? ins : ins < B3 ? ins - B1 : ins < B4 ? ins - B3 : ins - B4) * 64 + lane;
    if (ins < B1) {
      const int rg = P / C::CUP, u = P % C::CUP;  // rg = g * RT + row; u == CU: pad
      const int g = rg / RT, rr = rg % RT;
      const int row = row0 + rr;
      return P < C::WC && u < C::CU && row < N
                 ? codes_at + (uint32_t)row * (uint32_t)(nbr * C::CB) + (uint32_t)(g * SB * C::CB + 16 * u)
                 : kOOB;
    }
    if (ins < B3) {
      const int tg = P / C::AUP, u = P % C::AUP;
      const int g = tg / 16, t = tg % 16;
      return P < C::AC && u < SB * 16 && t < M ? (uint32_t)(t * K + g * SB * 256 + 16 * u) : kOOB;
    }
    if (ins < B4) {
      const int tg = P / (2 * SB), s = P % (2 * SB);
      const int g = tg / 16, t = tg % 16;
      return P < C::AS && t < M ? off_s + (uint32_t)((t * (K / 32) + g * SB * 8) * 4 + 16 * s) : kOOB;
    }
    if constexpr (QT == UB_Q4_K) {  // one dword per (group, super-block, token)
      const int gk = P / 16, t = P % 16;  // gk = g * SB + kbl
      return P < C::NDW && t < M ? off_d + (uint32_t)((t * nbr + gk) * 4) : kOOB;
    } else {
      const int tg = P / (2 * SB), s = P % (2 * SB);
      const int g = tg / 16, t = tg % 16;
      return P < KG * 16 * 2 * SB && t < M ? off_d + (uint32_t)((t * (K / 32) + g * SB * 8) * 4 + 16 * s)
                                           : kOOB;
    }
  };
  uint32_t lb[PW];
#pragma unroll
  for (int k = 0; k < PW; k++) {
    const int ins = k * NW + wv;
    lb[k] = ins < C::TI ? base_off(ins) : kOOB;
  }
  // Per load slot: LDS offset in a stage, per-step advance and kind (wave-
  // uniform).  Slots whose instructions all fall in one region for every
  // wavefront (known at compile time) take a branch-free path.
  uint32_t sl_lds[PW], sl_inc[PW];
  int sl_kind[PW];  // 0 weights, 1 activations (16 B), 2 activation scales (4 B), 3 none
#pragma unroll
  for (int k = 0; k < PW; k++) {
    const int ins = k * NW + wv;
    sl_lds[k] = ins < C::TI ? ins_lds(ins) : 0;
    sl_inc[k] = ins < C::TI ? ins_inc(ins) : 0;
    sl_kind[k] = ins >= C::TI ? 3 : ins < B1 ? 0 : (QT == UB_Q4_K && ins >= B4) ? 2 : 1;
  }
  // the last slot is real for the first TI - (PW - 1) NW wavefronts only
  const bool full_pw = (PW - 1) * NW + wv < C::TI;
  // Steps past the end load from offset 2^31 on: out of range for every lane.
  auto issue = [&](int st) {
    const uint32_t sb = ring0 + (uint32_t)((st % D) * C::SU * 16);
    const bool live = st < nsteps;
#pragma unroll
    for (int k = 0; k < PW; k++) {
      const int lo = k * NW, hi = lo + NW;  // instruction range of slot k
      const uint32_t soff = live ? (uint32_t)st * sl_inc[k] : 0x80000000u;
      const uint32_t la = sb + sl_lds[k];
      if (hi <= B1) {
        ub_lds_load16_at_nt(dw_, la, lb[k], soff);
      } else if (lo >= B1 && hi <= B3) {
        ub_lds_load16_at(da_, la, lb[k], soff);
      } else {
        const int kind = sl_kind[k];
        if (kind == 0) ub_lds_load16_at_nt(dw_, la, lb[k], soff);
        else if (kind == 1) ub_lds_load16_at(da_, la, lb[k], soff);
        else if (kind == 2) ub_lds_load4_at(da_, la, lb[k], soff);
        // kind 3: a slot past the step's instructions issues nothing
      }
    }
  };

  typedef int i32x4 __attribute__((ext_vector_type(4)));
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const i32x4 izero = {0, 0, 0, 0};
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  f32x4 mn = {0.f, 0.f, 0.f, 0.f};
  const int wrow = rw * 16 + r;  // this lane's row (A operand / headers) within the tile
  // Q4_0: the lane's nibble moved to the byte's high half (low nibbles for h < 2)
  const uint32_t nsh = 4u - 4u * (uint32_t)(h >> 1);

  // Block headers of the whole tile (16 B per row and 256 elements), once:
  // row r's headers are contiguous in memory, so the tile's are one run.  In
  // LDS row r starts at unit r (nbr + 1) (one pad unit: rows fall in distinct
  // banks); lanes on a pad unit or past the last row load nothing.  These
  // loads retire before the ring's first stage, which the first wait covers.
  {
    const int hu = RT * (nbr + 1);  // <= RT (HK + 1): every instruction lands inside hdr
    const int nrow = min(RT, N - row0);
    const uint32_t h0 = ub_lds_addr(hdr);
    for (int i = wv; i * 64 < hu; i += NW) {
      const int q = i * 64 + lane, rr = q / (nbr + 1), kb = q % (nbr + 1);
      const uint32_t off = rr < nrow && kb < nbr ? (uint32_t)((row0 + rr) * nbr + kb) * 16u : kOOB;
      ub_lds_load16_at_nt(dw_, h0 + (uint32_t)i * 1024, off, 0);
    }
  }
#pragma unroll
  for (int s = 0; s < D - 1; s++) issue(s);
  for (int st = 0; st < nsteps; st++) {
    // this wave's loads of step st have landed (PW or PW - 1 per step)
    if (full_pw) ub_wait_vmcnt<(D - 2) * PW>();
    else ub_wait_vmcnt<(D - 2) * (PW - 1)>();
    ub_barrier();                   // ... and every wave's; stage st-1 is free
    issue(st + D - 1);
    const uint32_t sb = ring0 + (uint32_t)((st % D) * C::SU * 16);
    // fragment bases: lane (row / token r, k-group h) reads 8 bytes at +8h of
    // each 32-byte run, so every read below is base + a constant
    uint32_t cbase = sb + (uint32_t)((C::oWC + (gw * RT + wrow) * C::CUP) * 16 +
                                     (QT == UB_Q4_0 ? 8 * (h & 1) : 8 * h));
    uint32_t abase = sb + (uint32_t)((C::oAC + (gw * 16 + r) * C::AUP) * 16 + 8 * h);
    // opaque to the compiler: one base register per region and step, the
    // constant parts of every read folded into ds_read offsets (otherwise it
    // keeps one register per read and rebases each of them every step)
    asm volatile("" : "+v"(cbase), "+v"(abase));
    if constexpr (QT == UB_Q4_K) {
      // Q4_K: activations are the A operand (row = token), weights the B
      // operand (column = weight row), so a lane owns one weight row r and
      // applies that row's sub-block scales from registers; its outputs are
      // tokens 4h..4h+3 of row r.
      const uint32_t hbase = ub_lds_addr(hdr) + (uint32_t)((wrow * (nbr + 1) + (st * KG + gw) * SB) * 16);
      uint32_t sbase = sb + (uint32_t)((C::oAS + (gw * 16 + r) * 2 * SB) * 16);
      uint32_t dbase = sb + (uint32_t)(C::oAD * 16 + gw * SB * 64);  // [kbl][token] dwords
      asm volatile("" : "+v"(sbase), "+v"(dbase));
#pragma unroll
      for (int kbl = 0; kbl < SB; kbl++) {
        const float dAr = __uint_as_float(ub_lds_read4(dbase + kbl * 64 + 4 * r));  // token r
        const uint4 dA4 = ub_lds_read16(dbase + kbl * 64 + 16 * h);  // tokens 4h..4h+3
        // header of row wrow: d | dmin, then the 6-bit scales / mins of the 8
        // sub-blocks packed in 12 bytes (get_scale_min_k4)
        const uint4 hd = ub_lds_read16(hbase + 16 * kbl);
        int sc[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          sc[j] = (hd.y >> (8 * j)) & 63;
          sc[4 + j] = ((hd.w >> (8 * j)) & 0xF) | (((hd.y >> (8 * j + 6)) & 3) << 4);
        }
        const uint32_t zb = (hd.z >> (8 * h)) & 0xff, wb = (hd.w >> (8 * h)) & 0xff;
        const int m0 = zb & 63, m1 = (wb >> 4) | ((zb >> 6) << 4);  // mins of sub-blocks h, 4 + h
        const float dw = ub_f16_to_f32((uint16_t)(hd.x & 0xffff));
        const float dmin = ub_f16_to_f32((uint16_t)(hd.x >> 16));
        // min term: A = d_a s_j (token r, k = h), B = dmin m_j (row r, k = h)
        const int sa0 = (int)ub_lds_read4(sbase + 4 * (kbl * 8 + h));
        const int sa1 = (int)ub_lds_read4(sbase + 4 * (kbl * 8 + 4 + h));
        mn = __builtin_amdgcn_mfma_f32_16x16x4f32(dAr * (float)sa0, dmin * (float)m0, mn, 0, 0, 0);
        mn = __builtin_amdgcn_mfma_f32_16x16x4f32(dAr * (float)sa1, dmin * (float)m1, mn, 0, 0, 0);
        i32x4 I[8];
#pragma unroll
        for (int p = 0; p < 4; p++) {
          // code bytes 32p + 8h.. (low nibbles: elements 64p + 8h.., high:
          // 64p + 32 + 8h..) and the matching activation elements
          const uint2 raw = ub_lds_read8(cbase + kbl * 128 + 32 * p);
          const uint2 b0 = ub_lds_read8(abase + kbl * 256 + 64 * p);
          const uint2 b1 = ub_lds_read8(abase + kbl * 256 + 64 * p + 32);
          const uint64_t lo = ((uint64_t)(raw.y & 0x0F0F0F0Fu) << 32) | (raw.x & 0x0F0F0F0Fu);
          const uint64_t hi = ((uint64_t)((raw.y >> 4) & 0x0F0F0F0Fu) << 32) | ((raw.x >> 4) & 0x0F0F0F0Fu);
          I[2 * p] = __builtin_amdgcn_mfma_i32_16x16x32_i8(
              (long)(((uint64_t)b0.y << 32) | b0.x), (long)lo, izero, 0, 0, 0);
          I[2 * p + 1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(
              (long)(((uint64_t)b1.y << 32) | b1.x), (long)hi, izero, 0, 0, 0);
        }
        // sum_j sc_j dot_j in integer (|dot| < 2^16, sc < 2^6: 24-bit products)
        int T[4] = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 8; j++) {
          T[0] += __mul24(sc[j], I[j][0]);
          T[1] += __mul24(sc[j], I[j][1]);
          T[2] += __mul24(sc[j], I[j][2]);
          T[3] += __mul24(sc[j], I[j][3]);
        }
        acc[0] += (dw * __uint_as_float(dA4.x)) * (float)T[0];
        acc[1] += (dw * __uint_as_float(dA4.y)) * (float)T[1];
        acc[2] += (dw * __uint_as_float(dA4.z)) * (float)T[2];
        acc[3] += (dw * __uint_as_float(dA4.w)) * (float)T[3];
      }
    } else {
      uint32_t dbase = sb + (uint32_t)((C::oAD + (gw * 16 + r) * 2 * SB) * 16);
      // headers of the lane's output rows 4h .. 4h + 3 (of the wave's 16)
      uint32_t obase = ub_lds_addr(hdr) + (uint32_t)(((rw * 16 + 4 * h) * (nbr + 1) + (st * KG + gw) * SB) * 16);
      const uint32_t rstr = (uint32_t)(nbr + 1) * 16;
      asm volatile("" : "+v"(dbase), "+v"(obase));
#pragma unroll
      for (int kbl = 0; kbl < SB; kbl++) {
        // the 8 fp16 block scales of each output row, used as fp16 operands
        // of v_fma_mix (no conversion instructions)
        uint4 hq[4];
#pragma unroll
        for (int i = 0; i < 4; i++) hq[i] = ub_lds_read16(obase + (uint32_t)i * rstr + 16 * kbl);
        constexpr float dsc = QT == UB_Q4_0 ? 0.0625f : 1.0f;  // exact power of two
        i32x4 I[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
          // elements 32j + 8h ..: Q8_0 codes; Q4_0 bytes 8 (h & 1) .. of the
          // block's 16, low nibbles for h < 2 (elements 0-15), high for the
          // rest, as the signed bytes 16 (q - 8) = (q << 4) ^ 0x80: the dot
          // is 16x the true one, and the block scale carries the 1/16
          uint2 av = ub_lds_read8(cbase + kbl * C::CB + (QT == UB_Q4_0 ? 16 : 32) * j);
          if constexpr (QT == UB_Q4_0) {
            av.x = ((av.x << nsh) & 0xF0F0F0F0u) ^ 0x80808080u;
            av.y = ((av.y << nsh) & 0xF0F0F0F0u) ^ 0x80808080u;
          }
          const uint2 bv = ub_lds_read8(abase + kbl * 256 + 32 * j);
          I[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(
              (long)(((uint64_t)av.y << 32) | av.x), (long)(((uint64_t)bv.y << 32) | bv.x), izero,
              0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
          // (d_w d_a) rounded once, as the f32 product of the converted d_w
          // and d_a (the 1/16 of Q4_0 moves to d_a exactly)
          const float dA = __uint_as_float(ub_lds_read4(dbase + 4 * (kbl * 8 + j))) * dsc;
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const uint32_t hw = (j >> 1) == 0 ? hq[i].x : (j >> 1) == 1 ? hq[i].y : (j >> 1) == 2 ? hq[i].z : hq[i].w;
            const _Float16 dw = __builtin_bit_cast(_Float16, (uint16_t)((j & 1) ? hw >> 16 : hw & 0xffff));
            const float t = __builtin_fmaf((float)dw, dA, 0.0f);
            acc[i] += t * (float)I[j][i];
          }
        }
      }
    }
  }
  ub_wait_vmcnt<0>();  // the trailing out-of-range loads still write the ring
  __syncthreads();     // every wave is done with the ring: it holds the partials now
  float* red = (float*)ring;
  static_assert(KG * 16 * RT * 4 <= D * C::SU * 16, "partials fit the ring");
  // partials [g][token][row] -> sum over groups in a fixed order, row-contiguous stores
  if constexpr (QT == UB_Q4_K) {  // lane: tokens 4h + i of row r
#pragma unroll
    for (int i = 0; i < 4; i++) red[(gw * 16 + 4 * h + i) * RT + rw * 16 + r] = acc[i] - mn[i];
  } else {  // lane: rows 4h + i, token r
    *(float4*)&red[(gw * 16 + r) * RT + rw * 16 + 4 * h] =
        make_float4(acc[0] - mn[0], acc[1] - mn[1], acc[2] - mn[2], acc[3] - mn[3]);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 16 * RT; i += 64 * NW) {
    const int t = i / RT, rr = i % RT;
    float v = red[t * RT + rr];
#pragma unroll
    for (int g = 1; g < KG; g++) v += red[(g * 16 + t) * RT + rr];
    if (t < M && row0 + rr < N) store_out<OT>(a.y, (size_t)t * N + row0 + rr, v);
  }
}

// LDS bytes of one k_gemv_mm workgroup (must stay within the CU's 160 KiB)
template <int QT, int RWV, int KG, int SB, int D, int HK>
constexpr int mm_lds() {
  using C = MmCfg<QT, RWV, KG, SB>;
  return D * C::SU * 16 + (C::RT * (HK + 1) + 63) / 64 * 64 * 16;
}

constexpr int kMmMaxSb = 128;  // longest row the ring GEMV takes: 128 x 256 elements

template <int QT, int OT, int RWV, int KG, int SB, int D, int HK>
void launch_mm_t(const GemvArgs& a, hipStream_t s) {
  const int nbr = a.K / 256;
  constexpr bool fits = mm_lds<QT, RWV, KG, SB, D, HK>() <= 160 * 1024;
  if constexpr (fits) {
    if (nbr % (KG * SB) == 0 && nbr <= HK)
      return k_gemv_mm<QT, OT, RWV, KG, SB, D, HK>
          <<<ub_cdiv(a.N, 16 * RWV), 64 * RWV * KG, 0, s>>>(a);
  }
  // (variants that do not fit this block type's LDS, or this K) any K up to
  // kMmMaxSb super-blocks
  k_gemv_mm<QT, OT, 1, 4, 1, 2, kMmMaxSb><<<ub_cdiv(a.N, 16), 256, 0, s>>>(a);
}

// Ring-GEMV variants <rows per workgroup / 16, K groups, super-blocks per
// group and step, ring depth, header capacity in super-blocks per row>;
// `cfg` from the gemv_mm knob, 0 = by shape: with N >= 16384 112-row tiles
// (N / 112 workgroups, about one per CU at the Llama-3-8B widths; 4-bit
// formats split K over two wavefront groups, which doubles the weight bytes
// in flight per workgroup: Q4_0 at 4096 x 28672 and 16 tokens 22.8 -> 20.1 us,
// while Q8_0's doubled stage no longer fits the LDS ring), below that
// 32- or 16-row tiles with K split over 4 or 8 wavefront groups so that a
// narrow matrix still spreads over the CUs (measured fastest on MI355X at the
// configs[1] shapes).
template <int QT, int OT>
void launch_mm(int cfg, const GemvArgs& a, hipStream_t s) {
  if (cfg <= 0) cfg = a.N >= 16384 ? (QT == UB_Q8_0 ? 1 : 13) : a.N > 4096 ? 5 : 7;
  switch (cfg) {
    case 1: return launch_mm_t<QT, OT, 7, 1, 1, 3, 16>(a, s);
    case 2: return launch_mm_t<QT, OT, 7, 1, 2, 2, 16>(a, s);
    case 3: return launch_mm_t<QT, OT, 4, 1, 1, 3, 16>(a, s);
    case 4: return launch_mm_t<QT, OT, 4, 1, 2, 2, 16>(a, s);
    case 5: return launch_mm_t<QT, OT, 2, 4, 1, 2, 56>(a, s);
    case 6: return launch_mm_t<QT, OT, 1, 4, 1, 3, 56>(a, s);
    case 7: return launch_mm_t<QT, OT, 1, 8, 1, 2, 56>(a, s);
    case 8: return launch_mm_t<QT, OT, 2, 2, 1, 3, 56>(a, s);
    case 9: return launch_mm_t<QT, OT, 1, 4, 1, 4, 56>(a, s);
    case 10: return launch_mm_t<QT, OT, 4, 2, 1, 2, 16>(a, s);
    case 11: return launch_mm_t<QT, OT, 7, 1, 1, 4, 16>(a, s);
    case 12: return launch_mm_t<QT, OT, 1, 2, 1, 4, 56>(a, s);
    case 13: return launch_mm_t<QT, OT, 7, 2, 1, 2, 16>(a, s);
    case 14: return launch_mm_t<QT, OT, 4, 2, 1, 3, 16>(a, s);
    case 15: return launch_mm_t<QT, OT, 4, 4, 1, 2, 16>(a, s);
    case 16: return launch_mm_t<QT, OT, 2, 8, 1, 2, 16>(a, s);
    case 17: return launch_mm_t<QT, OT, 7, 2, 1, 3, 16>(a, s);
    case 18: return launch_mm_t<QT, OT, 4, 4, 1, 3, 16>(a, s);
    case 19: return launch_mm_t<QT, OT, 2, 4, 1, 3, 56>(a, s);
    case 20: return launch_mm_t<QT, OT, 1, 8, 1, 3, 56>(a, s);
    case 21: return launch_mm_t<QT, OT, 7, 1, 1, 5, 16>(a, s);
    default: return launch_mm_t<QT, OT, 1, 4, 1, 2, kMmMaxSb>(a, s);
  }
}

// The ring GEMV takes a batch when K is a multiple of 1024 and every offset
// fits its 32-bit addressing (weights and workspace below 2 GiB).
bool mm_fits(int qt, const GemvArgs& a) {
  const size_t wb = a.nbw * (qt == UB_Q4_K ? 16 : 2) + (size_t)a.N * a.K / (qt == UB_Q8_0 ? 1 : 2);
  const size_t ab = (size_t)((const uint8_t*)a.sa - (const uint8_t*)a.qa) + (size_t)a.M * (a.K / 32) * 4;
  return a.K % 1024 == 0 && a.K / 256 <= kMmMaxSb && wb < (1ull << 31) && ab < (1ull << 31) &&
         a.K > 0;
}

template <int QT, int OT>
void launch_mfma(const GemvArgs& a, hipStream_t s) {
  const int w = ub_tune(UB_TUNE_GEMV_LDS_WAVES) == 4 ? 4 : 8;
  if (w == 8) k_gemv_mfma<QT, OT, 8><<<ub_cdiv(a.N, 16), 512, 0, s>>>(a);
  else k_gemv_mfma<QT, OT, 4><<<ub_cdiv(a.N, 16), 256, 0, s>>>(a);
}

// Q4_0 / Q8_0 rows longer than 8192 on matrices of at most 8192 rows, K %
// 1024 == 0: 3-4 tokens run the quantize launch + ring GEMV rather than the
// one-launch kernel (measured faster there; see ub_qmatmul).
bool q80_ring_first(int qt, int N, int K) {
  return qt != UB_Q4_K && K > 8192 && N <= 8192 && K % 1024 == 0;
}

template <int QT, int OT>
void launch_m(const GemvArgs& a, hipStream_t s) {
  {
    const int mm = ub_tune(UB_TUNE_GEMV_MFMA_M);  // fewest tokens for the MFMA path
    const int ring = ub_tune(UB_TUNE_GEMV_MM);  // ring GEMV: < 0 off, > 0 variant
    // From 3 tokens on wide matrices and where q80_ring_first holds (3-4
    // tokens there come from the two-launch QMatMul), from 5 elsewhere:
    // at 5-7 tokens on the narrow configs[1] shapes the ring measured (us,
    // single-pass kernels / ring) Q8_0 4096 x 4096 13.2-15.7 / 10.1-11.0,
    // Q4_0 4096 x 6144 13.5-16.5 / 10.2, Q4_K 4096 x 6144 12.5-13.4 / 9.6-9.7
    // (Q4_K 4096 x 4096 level).
    const bool wide = a.N >= 16384 || q80_ring_first(QT, a.N, a.K);
    const int ring_from = mm > 0 ? mm : (ring > 0 || wide ? 3 : 5);  // forced: 3
    if (ring >= 0 && a.M >= ring_from && a.M <= 16 && mm_fits(QT, a))
      return launch_mm<QT, OT>(ring, a, s);
  }
  if constexpr (QT == UB_Q8_0 || QT == UB_Q4_K) {
    const int mm = ub_tune(UB_TUNE_GEMV_MFMA_M);
    const int from = mm > 0 ? mm : (QT == UB_Q8_0 ? 17 : 5);
    if (a.M >= from && a.M <= 16) return launch_mfma<QT, OT>(a, s);
  }
  if (a.M <= 1) launch_ru<QT, 1, OT>(a, s);
  else if (a.M <= 2) launch_ru<QT, 2, OT>(a, s);
  else if (a.M <= 4) launch_ru<QT, 4, OT>(a, s);
  else if (a.M <= 8) launch_ru<QT, 8, OT>(a, s);
  else launch_ru<QT, 16, OT>(a, s);
}

template <int OT>
void launch_q(int qt, const GemvArgs& a, hipStream_t s) {
  if (qt == UB_Q4_0) launch_m<UB_Q4_0, OT>(a, s);
  else if (qt == UB_Q8_0) launch_m<UB_Q8_0, OT>(a, s);
  else launch_m<UB_Q4_K, OT>(a, s);
}

int check_args(int qt, const void* w, void* y, int M, int N, int K, const char* nm) {
  UB_REQUIRE(qt == UB_Q4_0 || qt == UB_Q8_0 || qt == UB_Q4_K, "%s: unsupported qtype %d", nm, qt);
  UB_REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative shape", nm);
  if ((size_t)M * N == 0) return UB_OK;
  UB_REQUIRE(w && y, "%s: null pointer", nm);
  int bk = qt == UB_Q4_K ? 256 : 32;
  UB_REQUIRE(K % bk == 0, "%s: K=%d is not a multiple of the block size %d", nm, K, bk);
  if (qt == UB_Q4_K) UB_REQUIRE(K % 256 == 0, "%s: K must be a multiple of 256", nm);
  size_t nbw = (size_t)N * K / bk;
  size_t head = qt == UB_Q4_K ? 16 : 2;
  UB_REQUIRE((((uintptr_t)w + nbw * head) & 15) == 0 && ((uintptr_t)w & 15) == 0,
             "%s: block payload must start 16-byte aligned (N*K/%d*%zu bytes of headers)", nm,
             bk, head);
  return UB_OK;
}

}  // namespace

// n 16-bit elements from x (2-byte aligned) to y, on s.
int ub_copy_b16(const void* x, void* y, size_t n, hipStream_t s) {
  if (n == 0) return UB_OK;
  k_b16_copy<<<(unsigned)std::min<size_t>((n + 255) / 256, 4096), 256, 0, s>>>(
      (const uint16_t*)x, (uint16_t*)y, n);
  return ub_check_launch("bf16 copy");
}

// ===================================================================== ABI
UB_API size_t ubridge_qmatmul_workspace_size(int qtype, int M, int K) {
  return qmm_ws_size(qtype, M, K);
}
// the same for ubridge_qmatmul_noalloc's routes
size_t ub_qmatmul_noalloc_ws(int qtype, int M, int K) { return qmm_ws_size(qtype, M, K, false); }

// Quantize activations x[M,K] (f32 or bf16) into the workspace in the
// weight's vec-dot format.  Split out so one quantization can feed several
// weights (e.g. Q, K, V of one token batch).
UB_API int ubridge_quantize_activations(int qtype, const void* x, int x_dtype, int M, int K,
                                        void* workspace, size_t ws_bytes, void* stream) {
  const char* nm = "ubridge_quantize_activations";
  if ((size_t)M * K == 0) return UB_OK;
  UB_REQUIRE(x && workspace, "%s: null pointer", nm);
  UB_REQUIRE(x_dtype == UB_F32 || x_dtype == UB_BF16, "%s: x_dtype %d (f32=0, bf16=2)", nm, x_dtype);
  UB_REQUIRE(ws_bytes >= ws_size(qtype, M, K), "%s: workspace %zu < %zu bytes", nm, ws_bytes,
             ws_size(qtype, M, K));
  int bk = qtype == UB_Q4_K ? 256 : 32;
  UB_REQUIRE(K % bk == 0, "%s: K=%d not a multiple of %d", nm, K, bk);
  if ((size_t)M * K == 0) return UB_OK;
  ActWs a = carve(workspace, qtype, M, K);
  hipStream_t s = ub_stream(stream);
  if (qtype == UB_Q4_K) return ub_quantize_act_q8_k(x, x_dtype, (size_t)M * K, a.q, a.d, a.s, s);
  if (qtype == UB_Q4_0 || qtype == UB_Q8_0)
    return ub_quantize_act_q8_0(x, x_dtype, (size_t)M * K, a.q, a.d, a.s, s);
  return ub_set_error(UB_ERR_UNSUPPORTED, "%s: qtype %d", nm, qtype);
}

// y[M,N] = x[M,K] . W[N,K]^T from activations already quantized into the
// workspace by ubridge_quantize_activations.  y_dtype f32 (0) or bf16 (2).
UB_API int ubridge_qmatmul_prequantized(int qtype, const void* w, void* y, int y_dtype, int M,
                                        int N, int K, const void* workspace, void* stream) {
  const char* nm = "ubridge_qmatmul_prequantized";
  int e = check_args(qtype, w, y, M, N, K, nm);
  if (e) return e;
  if (M == 0 || N == 0) return UB_OK;
  UB_REQUIRE(workspace || K == 0, "%s: null workspace", nm);
  UB_REQUIRE(y_dtype == UB_F32 || y_dtype == UB_BF16, "%s: y_dtype %d", nm, y_dtype);
  if (M == 0 || N == 0) return UB_OK;
  hipStream_t s = ub_stream(stream);
  for (int m0 = 0; m0 < M; m0 += 16) {
    int mc = M - m0 < 16 ? M - m0 : 16;
    ActWs a = carve(const_cast<void*>(workspace), qtype, M, K);
    a.q += (size_t)m0 * K;
    a.d += (size_t)m0 * K / (qtype == UB_Q4_K ? 256 : 32);
    a.s += (size_t)m0 * K / 32;
    size_t yo = (size_t)m0 * N * (y_dtype == UB_F32 ? 4 : 2);
    void* yc = (uint8_t*)y + yo;
    if (K == 0) {
      size_t nbytes = (size_t)mc * N * (y_dtype == UB_F32 ? 4 : 2);
      k_zero<<<ub_cdiv((long)nbytes, 256) < 4096 ? ub_cdiv((long)nbytes, 256) : 4096, 256, 0, s>>>(
          (uint8_t*)yc, nbytes);
      continue;
    }
    GemvArgs ga{(const uint8_t*)w, (size_t)N * K / (qtype == UB_Q4_K ? 256 : 32), a.q, a.d, a.s,
                yc, mc, N, K, nullptr};
    if (y_dtype == UB_F32) launch_q<UB_F32>(qtype, ga, s);
    else launch_q<UB_BF16>(qtype, ga, s);
  }
  return ub_check_launch(nm);
}

// One-call form: quantize x into the workspace, then the fused GEMV.  Up to
// 4 tokens (Q4_K: K <= 4096, else 2; Q4_0 / Q8_0: the LDS-staged kernel for K
// % 256 == 0 up to 16384, else 2 tokens with K <= 8192) a single kernel does
// both: each workgroup quantizes the activation chunk it needs into LDS
// while its weight loads are in flight (bit-identical codes to the
// two-launch form; the workspace is not touched).
// ubridge_qmatmul; may_alloc false keeps to the forms that allocate nothing
// (no library workspace, no hipBLASLt handle or plan): ubridge_qmatmul_noalloc.
int ub_qmatmul(int qtype, const void* w, const void* x, int x_dtype, void* y, int y_dtype, int M,
               int N, int K, void* workspace, size_t ws_bytes, void* stream, bool may_alloc);

UB_API int ubridge_qmatmul(int qtype, const void* w, const void* x, int x_dtype, void* y,
                           int y_dtype, int M, int N, int K, void* workspace, size_t ws_bytes,
                           void* stream) {
  return ub_qmatmul(qtype, w, x, x_dtype, y, y_dtype, M, N, K, workspace, ws_bytes, stream, true);
}

int ub_qmatmul(int qtype, const void* w, const void* x, int x_dtype, void* y, int y_dtype, int M,
               int N, int K, void* workspace, size_t ws_bytes, void* stream, bool may_alloc) {
  // The one-launch kernels read x with 16-byte loads; a misaligned x takes
  // the two-launch path below (same results), so alignment never decides
  // whether a valid call succeeds.
  const bool x_aligned = ((uintptr_t)x & 15) == 0;
  const int bk = qtype == UB_Q4_K ? 256 : 32;
  const int path = ub_tune(UB_TUNE_W4A16_PATH);
  // The pipelined MFMA GEMM that dequantizes in registers from LDS (no
  // slab) from qmm_fused_m tokens to where the slab route becomes faster; from
  // qmm_lib_m at every size when the call may not allocate (then without the
  // K split over workgroups); from 17 under knob w4a16_path = 4 (7: the same
  // without the K split; 2: never)
  if (may_alloc) ub_blaslt_prepare(ub_stream(stream));
  const bool fused = path == 4 || path == 7 ? M > 16
                     : path == 0 && (may_alloc ? M >= qmm_fused_m(qtype, N) && M < kGgufFusedHi
                                               : M >= qmm_lib_m(qtype));
  // The GEMM routes below read x as bf16 rows with 16-byte loads: f32 x, and
  // bf16 x that is not 16-byte aligned, are converted / copied once into the
  // caller's workspace (which has room for it from 17 tokens on) and every
  // GEMM route reads that copy.
  const bool gguf = qtype == UB_Q4_K || qtype == UB_Q8_0 || qtype == UB_Q4_0;
  const bool ws_copy = workspace && ((uintptr_t)workspace & 15) == 0 &&
                       ws_bytes >= (size_t)M * K * 2;
  const bool xb_ok = x && ((x_dtype == UB_BF16 && x_aligned) ||
                           ((x_dtype == UB_F32 || x_dtype == UB_BF16) && ws_copy));
  const bool gemm_args = gguf && xb_ok && N > 0 && K > 0 && w && y &&
                         (y_dtype == UB_F32 || y_dtype == UB_BF16);
  const void* xb = nullptr;
  auto bf16_x = [&](hipStream_t s) -> const void* {
    if (!xb) {
      if (x_dtype == UB_BF16 && x_aligned) {
        xb = x;
      } else {
        const size_t n = (size_t)M * K;
        const unsigned g = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
        if (x_dtype == UB_F32)
          k_f32_to_bf16<<<g, 256, 0, s>>>((const float*)x, (uint16_t*)workspace, n);
        else
          k_b16_copy<<<g, 256, 0, s>>>((const uint16_t*)x, (uint16_t*)workspace, n);
        xb = workspace;
      }
    }
    return xb;
  };
  if (gemm_args && fused && ub_gguf_pipelined_fits(qtype, M, N, K)) {
    hipStream_t s = ub_stream(stream);
    const int e = ub_gguf_pipelined(qtype, w, bf16_x(s), y, y_dtype == UB_F32, M, N, K, may_alloc, s);
    if (e != UB_ERR_UNSUPPORTED) return e;
  }
  if (gemm_args && M >= qmm_lib_m(qtype) && K % bk == 0 && path != 1 && may_alloc &&
      (size_t)M * K * 2 < 0x80000000ull) {
    hipStream_t s = ub_stream(stream);
    const int c32 = y_dtype == UB_F32;
    int slab = (int)std::min<size_t>((size_t)N, std::max<size_t>(256, kQmmSlabBytes / ((size_t)K * 2)));
    const int tail = N % slab;
    if (ub_blaslt_ready(1, M, slab, K, 1, 0, N, c32, UB_BF16, s) &&
        (tail == 0 || ub_blaslt_ready(1, M, tail, K, 1, 0, N, c32, UB_BF16, s))) {
      UbScratch ws(s, (size_t)slab * K * 2);
      void* scratch = ws.get();
      if (scratch) {
        const void* xs = bf16_x(s);
        for (int r0 = 0; r0 < N; r0 += slab) {
          const int nr = std::min(slab, N - r0);
          int e = ub_dequant_rows(qtype, w, N, K, r0, nr, scratch, UB_BF16, s);
          if (e) return e;
          e = ub_blaslt_gemm(xs, scratch, (uint8_t*)y + (size_t)r0 * (c32 ? 4 : 2), 1, M, nr, K, 1,
                             0, N, c32, UB_BF16, s);
          if (e) return ub_set_error(e == UB_ERR_UNSUPPORTED ? UB_ERR_LAUNCH : e,
                                     "ubridge_qmatmul: library GEMM of a slab failed");
        }
        return ub_check_launch("ubridge_qmatmul");
      }
    }
  }
  if (gemm_args && M >= kQmmGemmM) {
    hipStream_t s = ub_stream(stream);
    const int e = ub_gguf_gemm(qtype, w, bf16_x(s), y, y_dtype == UB_F32, M, N, K, s);
    if (e != UB_ERR_UNSUPPORTED) return e ? e : ub_check_launch("ubridge_qmatmul");
  }
  // One launch (activations quantized per workgroup in LDS while its weight
  // loads fly) up to fuse_m tokens; beyond, a quantize launch + the GEMV.
  // Measured on MI355X (configs[1] shapes, us, two launches / one): Q8_0 3-4
  // tokens 4096 x 28672 30.1 / 23.2, 4096 x 6144 12.2 / 8.7; Q4_K 4096 x 6144
  // 4 tokens 9.75 / 9.22, 4096 x 28672 (persistent grid with rolling
  // prefetch) 3 tokens 18.6 / 15.4, 4 tokens 18.5 / 17.9 -- one launch up to
  // 4 tokens for K <= 4096.  Beyond: Q4_0 / Q8_0 at 3-4 tokens on rows
  // longer than 8192 (the one-launch kernel walks K in four chunks) lose to
  // the quantize launch + ring GEMV on narrow matrices: 14336 x 4096 Q8_0
  // 18.4 / 20.7 -> 17.8 / 17.9, Q4_0 15.7 / 18.1 -> 14.3 / 14.3; but not at
  // 8192 x 4096 (Q8_0 3 tokens 11.8 one launch, 13.7 two) nor on wide ones
  // (8192 x 14336 22.8 / 35.6).  Q4_K at 2 tokens: two launches from K = 8192
  // or N = 8192 (8192 x 14336 21.8 -> 18.2, 14336 x 4096 12.6 -> 11.8,
  // 5120 x 14336 18.2 -> 17.4), one at 5120 x 4096 (6.9 against 8.2); Q4_K
  // 3-4 tokens stay two launches beyond K = 4096 (14336 x 4096 3 tokens 13.4
  // against 16.5).
  const int fuse_knob = ub_tune(UB_TUNE_GEMV_FUSE_M);
  const bool q4k_long = K >= 8192 || N >= 8192;
  const int fuse_m = fuse_knob > 0                  ? std::min(fuse_knob, 4)
                     : K <= 4096                    ? 4
                     : qtype == UB_Q4_K             ? (q4k_long ? 1 : 2)
                     : q80_ring_first(qtype, N, K) ? 2
                                                    : 4;
  if (qtype == UB_Q4_K && M >= 1 && M <= fuse_m && N > 0 && K > 0 && x_aligned && lds_enabled()) {
    const char* nm = "ubridge_qmatmul";
    int e = check_args(qtype, w, y, M, N, K, nm);
    if (e) return e;
    UB_REQUIRE(x, "%s: null pointer", nm);
    UB_REQUIRE(x_dtype == UB_F32 || x_dtype == UB_BF16, "%s: x_dtype %d (f32=0, bf16=2)", nm,
               x_dtype);
    UB_REQUIRE(y_dtype == UB_F32 || y_dtype == UB_BF16, "%s: y_dtype %d", nm, y_dtype);
    UB_REQUIRE(ws_bytes >= ws_size(qtype, M, K) && workspace, "%s: workspace %zu < %zu bytes",
               nm, ws_bytes, ws_size(qtype, M, K));
    GemvArgs ga{(const uint8_t*)w, (size_t)N * K / 256, nullptr, nullptr, nullptr, y, M, N, K, x};
    hipStream_t s = ub_stream(stream);
    if (M == 1) {
      if (y_dtype == UB_F32) {
        if (x_dtype == UB_F32) launch_lds_r<1, UB_F32, UB_F32>(ga, s);
        else launch_lds_r<1, UB_F32, UB_BF16>(ga, s);
      } else {
        if (x_dtype == UB_F32) launch_lds_r<1, UB_BF16, UB_F32>(ga, s);
        else launch_lds_r<1, UB_BF16, UB_BF16>(ga, s);
      }
    } else if (M == 2) {
      if (y_dtype == UB_F32) {
        if (x_dtype == UB_F32) launch_lds_r<2, UB_F32, UB_F32>(ga, s);
        else launch_lds_r<2, UB_F32, UB_BF16>(ga, s);
      } else {
        if (x_dtype == UB_F32) launch_lds_r<2, UB_BF16, UB_F32>(ga, s);
        else launch_lds_r<2, UB_BF16, UB_BF16>(ga, s);
      }
    } else {
      if (y_dtype == UB_F32) {
        if (x_dtype == UB_F32) launch_lds_r<4, UB_F32, UB_F32>(ga, s);
        else launch_lds_r<4, UB_F32, UB_BF16>(ga, s);
      } else {
        if (x_dtype == UB_F32) launch_lds_r<4, UB_BF16, UB_F32>(ga, s);
        else launch_lds_r<4, UB_BF16, UB_BF16>(ga, s);
      }
    }
    return ub_check_launch(nm);
  }
  const bool q80_lds = K % 256 == 0 && K <= 16384 && ub_tune(UB_TUNE_GEMV_Q80_LDS) >= 0;
  if ((qtype == UB_Q4_0 || qtype == UB_Q8_0) && M >= 1 && N > 0 && K > 0 &&
      ((M <= 2 && (K <= kFusedMaxK || q80_lds)) || (M <= fuse_m && q80_lds)) && x_aligned) {
    // Q4_0 / Q8_0, 1-4 tokens: one kernel quantizes x per workgroup and runs
    // the GEMV (bit-identical codes to the two-launch form); 3-4 tokens on
    // the LDS-staged form only
    const char* nm = "ubridge_qmatmul";
    int e = check_args(qtype, w, y, M, N, K, nm);
    if (e) return e;
    UB_REQUIRE(x, "%s: null pointer", nm);
    UB_REQUIRE(x_dtype == UB_F32 || x_dtype == UB_BF16, "%s: x_dtype %d (f32=0, bf16=2)", nm,
               x_dtype);
    UB_REQUIRE(y_dtype == UB_F32 || y_dtype == UB_BF16, "%s: y_dtype %d", nm, y_dtype);
    UB_REQUIRE(ws_bytes >= ws_size(qtype, M, K) && workspace, "%s: workspace %zu < %zu bytes",
               nm, ws_bytes, ws_size(qtype, M, K));
    GemvArgs ga{(const uint8_t*)w, (size_t)N * K / 32, nullptr, nullptr, nullptr, y, M, N, K, x};
    hipStream_t s = ub_stream(stream);
    if (qtype == UB_Q4_0) launch_fused_q80_t<UB_Q4_0>(x_dtype, y_dtype, ga, s);
    else launch_fused_q80_t<UB_Q8_0>(x_dtype, y_dtype, ga, s);
    return ub_check_launch(nm);
  }
  int e = ubridge_quantize_activations(qtype, x, x_dtype, M, K, workspace, ws_bytes, stream);
  if (e) return e;
  return ubridge_qmatmul_prequantized(qtype, w, y, y_dtype, M, N, K, workspace, stream);
}

