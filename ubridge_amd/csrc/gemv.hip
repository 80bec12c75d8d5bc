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

int ub_quantize_act_q8_0(const void* x, int x_dt, size_t n, int8_t* q, float* d, int* s,
                         hipStream_t st);
int ub_quantize_act_q8_k(const void* x, int x_dt, size_t n, int8_t* q, float* d, int* bs,
                         hipStream_t st);

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
// log2 NV) shuffles instead of 6*NV.  Afterwards lane L holds the wave total
// of value index L >> (6 - log2 NV) in v[0].
template <int NV>
__device__ __forceinline__ float wave_reduce_scatter(float (&v)[NV], int lane) {
  static_assert(NV >= 1 && NV <= 64 && (NV & (NV - 1)) == 0, "NV must be a power of two <= 64");
#pragma unroll
  for (int step = 0; step < 6; step++) {
    const int off = 32 >> step;
    const int c = (NV >> step) > 1 ? (NV >> step) : 1;
    if (c > 1) {
      const bool upper = (lane & off) != 0;
#pragma unroll
      for (int i = 0; i < c / 2; i++) {
        float send = upper ? v[i] : v[i + c / 2];
        float keep = upper ? v[i + c / 2] : v[i];
        v[i] = keep + __shfl_xor(send, off, 64);
      }
    } else {
      v[0] += __shfl_xor(v[0], off, 64);
    }
  }
  return v[0];
}

template <int N>
constexpr int ilog2() { return N <= 1 ? 0 : 1 + ilog2<N / 2>(); }

// ----------------------------------------------------------- block codecs
// Q4_0 / Q8_0: one lane per 32-element block.  Q4_0: 16 code bytes (low
// nibbles of dword i = elements 4i..4i+3, high nibbles 16+4i..), and
// sum (q-8)*a = sum q*a - 8*sum a with the per-block activation code sum.
// Q4_K: four lanes (a quad) per 256-element super-block; lane t = lane%4 reads
// code bytes [32t, 32t+32): their low nibbles are elements 64t+(0..31)
// (sub-block 2t), their high nibbles 64t+32+(0..31) (sub-block 2t+1).  Per
// block and token:
//   d_w*d_a*(sc_lo*dot_lo + sc_hi*dot_hi) - dmin_w*d_a*(m_lo*s_lo + m_hi*s_hi)
// with s the 32-element activation code sums.
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
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  u32x4b v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kAuxNT);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t bload4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t bload2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}

template <int K>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K | (K << 2) | (K << 4) | (K << 6), 0xf, 0xf,
                                            false);
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
__device__ __forceinline__ int dot_hi(const uint4& w, const uint4& a, int s) {
  s = dot4((w.x >> 4) & 0x0F0F0F0Fu, a.x, s);
  s = dot4((w.y >> 4) & 0x0F0F0F0Fu, a.y, s);
  s = dot4((w.z >> 4) & 0x0F0F0F0Fu, a.z, s);
  return dot4((w.w >> 4) & 0x0F0F0F0Fu, a.w, s);
}
__device__ __forceinline__ int dot_i8(const uint4& w, const uint4& a, int s) {
  s = dot4(w.x, a.x, s);
  s = dot4(w.y, a.y, s);
  s = dot4(w.z, a.z, s);
  return dot4(w.w, a.w, s);
}

// 6-bit scales / mins of sub-blocks 2t and 2t+1 (get_scale_min_k4,
// quant.cpp:356-363), from the three scale dwords d1..d3 of the header
// (bytes 4..15).  For t < 2 both sub-blocks are < 4: sc = byte[s] & 63,
// m = byte[s+4] & 63; for t >= 2 they are >= 4 and take their low 4 bits from
// byte[s+4] and their top 2 bits from byte[s-4] / byte[s].  With u = t & 1
// the needed bytes sit at bit 16u of each dword.
__device__ __forceinline__ void q4k_scales(int t, uint32_t d1, uint32_t d2, uint32_t d3, int& sc0,
                                           int& sc1, int& m0, int& m1) {
  const int sh = (t & 1) * 16;
  const uint32_t e1 = d1 >> sh, e2 = d2 >> sh, e3 = d3 >> sh;
  if (t < 2) {
    sc0 = e1 & 63;
    sc1 = (e1 >> 8) & 63;
    m0 = e2 & 63;
    m1 = (e2 >> 8) & 63;
  } else {
    sc0 = (e3 & 0xF) | (((e1 >> 6) & 3) << 4);
    sc1 = ((e3 >> 8) & 0xF) | (((e1 >> 14) & 3) << 4);
    m0 = ((e3 >> 4) & 0xF) | (((e2 >> 6) & 3) << 4);
    m1 = ((e3 >> 12) & 0xF) | (((e2 >> 14) & 3) << 4);
  }
}

struct GemvArgs {
  const uint8_t* w;
  size_t nbw;
  const int8_t* qa;
  const float* da;
  const int* sa;
  void* y;
  int M, N, K;
};

// ------------------------------------------------------------ GEMV kernel
// A wavefront owns R consecutive rows and issues the loads of U
// block-iterations x R rows before any arithmetic; the activations of those
// blocks are then read once from L1/L2 and reused across the R rows.
template <int QT, int MT, int R, int U, int OT>
__global__ void __launch_bounds__(256) k_gemv(GemvArgs a) {
  using G = Geo<QT>;
  const int lane = threadIdx.x & 63;
  // wave-uniform (scalar) row index, so the buffer descriptors live in SGPRs
  const int row0 = (blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * R;
  if (row0 >= a.N) return;
  const int nbr = a.K / G::BK;
  const int kb0 = lane / G::LPB, t = lane % G::LPB;
  const int M = a.M, N = a.N, K = a.K;
  const int nrows = min(R, N - row0);
  const __amdgpu_buffer_rsrc_t rq =
      rsrc(a.w + a.nbw * G::HB + (size_t)row0 * nbr * G::QB, (uint32_t)(nrows * nbr * G::QB));
  const __amdgpu_buffer_rsrc_t rh =
      rsrc(a.w + (size_t)row0 * nbr * G::HB, (uint32_t)(nrows * nbr * G::HB));

  float acc[R * MT];
#pragma unroll
  for (int i = 0; i < R * MT; i++) acc[i] = 0.f;

  for (int it = 0; it * G::BPI < nbr; it += U) {
    WReg wr[U][R];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int kb = kb0 + (it + u) * G::BPI;
#pragma unroll
      for (int r = 0; r < R; r++)
        load_w<QT>(wr[u][r], rq, rh, (uint32_t)(r * nbr + kb), kb < nbr, t);
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int kb = min(kb0 + (it + u) * G::BPI, nbr - 1);  // clamped: activations stay in bounds
      if constexpr (QT == UB_Q4_K) {
        int sc0[R], sc1[R], mn0[R], mn1[R];
        float dw[R], dm[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
          const uint32_t hv = wr[u][r].h;
          const uint32_t h0 = quad_bcast<0>(hv), h1 = quad_bcast<1>(hv), h2 = quad_bcast<2>(hv),
                         h3 = quad_bcast<3>(hv);
          q4k_scales(t, h1, h2, h3, sc0[r], sc1[r], mn0[r], mn1[r]);
          dw[r] = ub_f16_to_f32((uint16_t)(h0 & 0xffff));
          dm[r] = ub_f16_to_f32((uint16_t)(h0 >> 16));
        }
#pragma unroll
        for (int m = 0; m < MT; m++) {
          if (MT == 1 || m < M) {
            const uint4* ab = (const uint4*)(a.qa + (size_t)m * K + (size_t)kb * 256 + 64 * t);
            const uint4 al0 = ab[0], al1 = ab[1], ah0 = ab[2], ah1 = ab[3];
            const int2 ss = *(const int2*)(a.sa + (size_t)m * (K >> 5) + (size_t)kb * 8 + 2 * t);
            const float dam = a.da[(size_t)m * nbr + kb];
#pragma unroll
            for (int r = 0; r < R; r++) {
              const int slo = dot_lo(wr[u][r].q1, al1, dot_lo(wr[u][r].q0, al0, 0));
              const int shi = dot_hi(wr[u][r].q1, ah1, dot_hi(wr[u][r].q0, ah0, 0));
              const int isum = sc0[r] * slo + sc1[r] * shi;
              const int imin = mn0[r] * ss.x + mn1[r] * ss.y;
              acc[r * MT + m] += (dw[r] * dam) * (float)isum - (dm[r] * dam) * (float)imin;
            }
          }
        }
      } else {
#pragma unroll
        for (int m = 0; m < MT; m++) {
          if (MT == 1 || m < M) {
            const uint4* ap = (const uint4*)(a.qa + (size_t)m * K + (size_t)kb * 32);
            const uint4 a0 = ap[0], a1 = ap[1];
            const float dam = a.da[(size_t)m * nbr + kb];
            int sam = 0;
            if constexpr (QT == UB_Q4_0) sam = a.sa[(size_t)m * nbr + kb];
#pragma unroll
            for (int r = 0; r < R; r++) {
              int s;
              if constexpr (QT == UB_Q4_0)
                s = dot_hi(wr[u][r].q0, a1, dot_lo(wr[u][r].q0, a0, 0)) - 8 * sam;
              else
                s = dot_i8(wr[u][r].q1, a1, dot_i8(wr[u][r].q0, a0, 0));
              // an out-of-range block reads d = 0 and adds nothing
              acc[r * MT + m] += (float)s * ub_f16_to_f32((uint16_t)wr[u][r].h) * dam;
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

template <int QT, int MT, int R, int U, int OT>
void launch_t(const GemvArgs& a, hipStream_t s) {
  k_gemv<QT, MT, R, U, OT><<<ub_cdiv(a.N, kWaves * R), 256, 0, s>>>(a);
}

int env_int(const char* n) {
  const char* v = getenv(n);
  return v ? atoi(v) : 0;
}

// Rows per wavefront (R) and block-iterations per pass (U), from a sweep of
// the Llama-3-8B decode shapes on MI355X: R = 2 keeps ~8 KiB in flight per
// wavefront without cutting occupancy; R = 4 only pays for the widest Q4_K
// layers at M = 1; U = 2 only for Q4_K with >= 2 iterations (K >= 8192).
// UBRIDGE_GEMV_R / UBRIDGE_GEMV_U override the choice (tuning runs).
template <int QT, int MT, int OT>
void launch_ru(const GemvArgs& a, hipStream_t s) {
  using G = Geo<QT>;
  static const int env_r = env_int("UBRIDGE_GEMV_R"), env_u = env_int("UBRIDGE_GEMV_U");
  const int iters = (a.K / G::BK + G::BPI - 1) / G::BPI;
  int r = 2;
  if (QT == UB_Q4_K && MT == 1 && a.N >= 16384) r = 4;
  if (QT == UB_Q8_0 && a.N < 8192 && MT == 1) r = 1;
  if (env_r) r = env_r;
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

template <int QT, int OT>
void launch_m(const GemvArgs& a, hipStream_t s) {
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

// ===================================================================== ABI
UB_API size_t ubridge_qmatmul_workspace_size(int qtype, int M, int K) {
  return ws_size(qtype, M, K);
}

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
                yc, mc, N, K};
    if (y_dtype == UB_F32) launch_q<UB_F32>(qtype, ga, s);
    else launch_q<UB_BF16>(qtype, ga, s);
  }
  return ub_check_launch(nm);
}

// One-call form: quantize x into the workspace, then the fused GEMV.
UB_API int ubridge_qmatmul(int qtype, const void* w, const void* x, int x_dtype, void* y,
                           int y_dtype, int M, int N, int K, void* workspace, size_t ws_bytes,
                           void* stream) {
  int e = ubridge_quantize_activations(qtype, x, x_dtype, M, K, workspace, ws_bytes, stream);
  if (e) return e;
  return ubridge_qmatmul_prequantized(qtype, w, y, y_dtype, M, N, K, workspace, stream);
}
