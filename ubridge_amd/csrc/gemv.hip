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
  int* s;  // Q8_0: per-32 code sums; Q8_K: per-16 code sums
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
  if (qt == UB_Q4_K) return al256(n) + al256(4 * (n / 256)) + al256(4 * (n / 16));
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

// ------------------------------------------------------------------ Q4_0
// Lane owns block kb of each row: 16 code bytes = 4 dwords; low nibbles of
// dword i are elements 4i..4i+3, high nibbles 16+4i..16+4i+3.
// sum (q-8)*a = sum q*a - 8*sum a, with sum a precomputed per block.
template <int MT, int R, int OT>
__global__ void __launch_bounds__(256) k_gemv_q4_0(const uint8_t* __restrict__ w, size_t nbw,
                                                   const int8_t* __restrict__ qa,
                                                   const float* __restrict__ da,
                                                   const int* __restrict__ sa,
                                                   void* __restrict__ y, int M, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * R;
  if (row0 >= N) return;
  const int nbr = K >> 5;
  const uint16_t* wd = (const uint16_t*)w;
  const uint4* wq = (const uint4*)(w + nbw * 2);
  float acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int m = 0; m < MT; m++) acc[r][m] = 0.f;

  for (int kb = lane; kb < nbr; kb += 64) {
    uint4 q[R];
    float dw[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      int n = min(row0 + r, N - 1);
      size_t b = (size_t)n * nbr + kb;
      q[r] = ld_nt(&wq[b]);
      dw[r] = ub_f16_to_f32(wd[b]);
    }
#pragma unroll
    for (int m = 0; m < MT; m++) {
      if (m < M) {
        const uint4* ap = (const uint4*)(qa + (size_t)m * K + (size_t)kb * 32);
        uint4 a0 = ap[0], a1 = ap[1];
        float dam = da[(size_t)m * nbr + kb];
        int sam = sa[(size_t)m * nbr + kb];
#pragma unroll
        for (int r = 0; r < R; r++) {
          uint32_t w0 = q[r].x, w1 = q[r].y, w2 = q[r].z, w3 = q[r].w;
          int s = 0;
          s = dot4(w0 & 0x0F0F0F0Fu, a0.x, s);
          s = dot4(w1 & 0x0F0F0F0Fu, a0.y, s);
          s = dot4(w2 & 0x0F0F0F0Fu, a0.z, s);
          s = dot4(w3 & 0x0F0F0F0Fu, a0.w, s);
          s = dot4((w0 >> 4) & 0x0F0F0F0Fu, a1.x, s);
          s = dot4((w1 >> 4) & 0x0F0F0F0Fu, a1.y, s);
          s = dot4((w2 >> 4) & 0x0F0F0F0Fu, a1.z, s);
          s = dot4((w3 >> 4) & 0x0F0F0F0Fu, a1.w, s);
          s -= 8 * sam;
          acc[r][m] += (float)s * dw[r] * dam;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int m = 0; m < MT; m++) {
      float v = ub_wave_sum(acc[r][m]);
      if (lane == 0 && m < M && row0 + r < N) store_out<OT>(y, (size_t)m * N + row0 + r, v);
    }
}

// ------------------------------------------------------------------ Q8_0
template <int MT, int R, int OT>
__global__ void __launch_bounds__(256) k_gemv_q8_0(const uint8_t* __restrict__ w, size_t nbw,
                                                   const int8_t* __restrict__ qa,
                                                   const float* __restrict__ da,
                                                   void* __restrict__ y, int M, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * R;
  if (row0 >= N) return;
  const int nbr = K >> 5;
  const uint16_t* wd = (const uint16_t*)w;
  const uint4* wq = (const uint4*)(w + nbw * 2);
  float acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int m = 0; m < MT; m++) acc[r][m] = 0.f;

  for (int kb = lane; kb < nbr; kb += 64) {
    uint4 q0[R], q1[R];
    float dw[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      int n = min(row0 + r, N - 1);
      size_t b = (size_t)n * nbr + kb;
      q0[r] = ld_nt(&wq[2 * b]);
      q1[r] = ld_nt(&wq[2 * b + 1]);
      dw[r] = ub_f16_to_f32(wd[b]);
    }
#pragma unroll
    for (int m = 0; m < MT; m++) {
      if (m < M) {
        const uint4* ap = (const uint4*)(qa + (size_t)m * K + (size_t)kb * 32);
        uint4 a0 = ap[0], a1 = ap[1];
        float dam = da[(size_t)m * nbr + kb];
#pragma unroll
        for (int r = 0; r < R; r++) {
          int s = 0;
          s = dot4(q0[r].x, a0.x, s);
          s = dot4(q0[r].y, a0.y, s);
          s = dot4(q0[r].z, a0.z, s);
          s = dot4(q0[r].w, a0.w, s);
          s = dot4(q1[r].x, a1.x, s);
          s = dot4(q1[r].y, a1.y, s);
          s = dot4(q1[r].z, a1.z, s);
          s = dot4(q1[r].w, a1.w, s);
          acc[r][m] += (float)s * dw[r] * dam;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int m = 0; m < MT; m++) {
      float v = ub_wave_sum(acc[r][m]);
      if (lane == 0 && m < M && row0 + r < N) store_out<OT>(y, (size_t)m * N + row0 + r, v);
    }
}

// ------------------------------------------------------------------ Q4_K
__device__ __forceinline__ int byte_of(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
  uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
  return (int)((w >> (8 * (i & 3))) & 0xff);
}
// get_scale_min_k4 (quant.cpp:356-363).
__device__ __forceinline__ void scale_min(int s, uint32_t s0, uint32_t s1, uint32_t s2, int& sc,
                                          int& mn) {
  if (s < 4) {
    sc = byte_of(s0, s1, s2, s) & 63;
    mn = byte_of(s0, s1, s2, s + 4) & 63;
  } else {
    sc = (byte_of(s0, s1, s2, s + 4) & 0xF) | ((byte_of(s0, s1, s2, s - 4) >> 6) << 4);
    mn = (byte_of(s0, s1, s2, s + 4) >> 4) | ((byte_of(s0, s1, s2, s) >> 6) << 4);
  }
}

// Eight lanes per 256-element super-block; lane t = lane%8 reads code bytes
// [16t, 16t+16): group j = t/2, half h = t%2, low nibbles are elements
// 64j+16h+(0..15) of sub-block 2j, high nibbles 64j+32+16h+(0..15) of
// sub-block 2j+1.  Per block and token:
//   d_w*d_a*(sc_lo*dot_lo + sc_hi*dot_hi) - dmin_w*d_a*(m_lo*bs_lo + m_hi*bs_hi)
// with bs the 16-element activation code sums.
template <int MT, int R, int OT>
__global__ void __launch_bounds__(256) k_gemv_q4_k(const uint8_t* __restrict__ w, size_t nbw,
                                                   const int8_t* __restrict__ qa,
                                                   const float* __restrict__ da,
                                                   const int* __restrict__ bsum,
                                                   void* __restrict__ y, int M, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * R;
  if (row0 >= N) return;
  const int nbr = K >> 8;
  const int t = lane & 7, j = t >> 1, h = t & 1;
  const uint4* hdr = (const uint4*)w;
  const uint4* wq = (const uint4*)(w + nbw * 16);
  float acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int m = 0; m < MT; m++) acc[r][m] = 0.f;

  for (int kb = lane >> 3; kb < nbr; kb += 8) {
    uint4 q[R], hd[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      int n = min(row0 + r, N - 1);
      size_t b = (size_t)n * nbr + kb;
      q[r] = ld_nt(&wq[b * 8 + t]);
      hd[r] = hdr[b];
    }
    int sc0[R], sc1[R], mn0[R], mn1[R];
    float dw[R], dm[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      scale_min(2 * j, hd[r].y, hd[r].z, hd[r].w, sc0[r], mn0[r]);
      scale_min(2 * j + 1, hd[r].y, hd[r].z, hd[r].w, sc1[r], mn1[r]);
      dw[r] = ub_f16_to_f32((uint16_t)(hd[r].x & 0xffff));
      dm[r] = ub_f16_to_f32((uint16_t)(hd[r].x >> 16));
    }
#pragma unroll
    for (int m = 0; m < MT; m++) {
      if (m < M) {
        const int8_t* ab = qa + (size_t)m * K + (size_t)kb * 256 + 64 * j + 16 * h;
        uint4 alo = *(const uint4*)ab;
        uint4 ahi = *(const uint4*)(ab + 32);
        const int* bsp = bsum + (size_t)m * (K >> 4) + (size_t)kb * 16 + 4 * j + h;
        int bs_lo = bsp[0], bs_hi = bsp[2];
        float dam = da[(size_t)m * nbr + kb];
#pragma unroll
        for (int r = 0; r < R; r++) {
          uint32_t w0 = q[r].x, w1 = q[r].y, w2 = q[r].z, w3 = q[r].w;
          int slo = 0, shi = 0;
          slo = dot4(w0 & 0x0F0F0F0Fu, alo.x, slo);
          slo = dot4(w1 & 0x0F0F0F0Fu, alo.y, slo);
          slo = dot4(w2 & 0x0F0F0F0Fu, alo.z, slo);
          slo = dot4(w3 & 0x0F0F0F0Fu, alo.w, slo);
          shi = dot4((w0 >> 4) & 0x0F0F0F0Fu, ahi.x, shi);
          shi = dot4((w1 >> 4) & 0x0F0F0F0Fu, ahi.y, shi);
          shi = dot4((w2 >> 4) & 0x0F0F0F0Fu, ahi.z, shi);
          shi = dot4((w3 >> 4) & 0x0F0F0F0Fu, ahi.w, shi);
          int isum = sc0[r] * slo + sc1[r] * shi;
          int imin = mn0[r] * bs_lo + mn1[r] * bs_hi;
          acc[r][m] += (dw[r] * dam) * (float)isum - (dm[r] * dam) * (float)imin;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int m = 0; m < MT; m++) {
      float v = ub_wave_sum(acc[r][m]);
      if (lane == 0 && m < M && row0 + r < N) store_out<OT>(y, (size_t)m * N + row0 + r, v);
    }
}

template <int MT, int R, int OT>
void launch_t(int qt, const uint8_t* w, const ActWs& a, void* y, int M, int N, int K,
              hipStream_t s) {
  int grid = ub_cdiv(N, kWaves * R);
  size_t nbw = (size_t)N * K / (qt == UB_Q4_K ? 256 : 32);
  if (qt == UB_Q4_0)
    k_gemv_q4_0<MT, R, OT><<<grid, 256, 0, s>>>(w, nbw, a.q, a.d, a.s, y, M, N, K);
  else if (qt == UB_Q8_0)
    k_gemv_q8_0<MT, R, OT><<<grid, 256, 0, s>>>(w, nbw, a.q, a.d, y, M, N, K);
  else
    k_gemv_q4_k<MT, R, OT><<<grid, 256, 0, s>>>(w, nbw, a.q, a.d, a.s, y, M, N, K);
}

template <int MT, int OT>
void launch_r(int qt, const uint8_t* w, const ActWs& a, void* y, int M, int N, int K,
              hipStream_t s) {
  // Keep >= ~4096 wavefronts in flight (16 per CU) before grouping rows.
  int r = N >= 4 * 4096 ? 4 : (N >= 2 * 4096 ? 2 : 1);
  if (r == 4) launch_t<MT, 4, OT>(qt, w, a, y, M, N, K, s);
  else if (r == 2) launch_t<MT, 2, OT>(qt, w, a, y, M, N, K, s);
  else launch_t<MT, 1, OT>(qt, w, a, y, M, N, K, s);
}

template <int OT>
void launch_m(int qt, const uint8_t* w, const ActWs& a, void* y, int M, int N, int K,
              hipStream_t s) {
  if (M <= 1) launch_r<1, OT>(qt, w, a, y, M, N, K, s);
  else if (M <= 2) launch_r<2, OT>(qt, w, a, y, M, N, K, s);
  else if (M <= 4) launch_r<4, OT>(qt, w, a, y, M, N, K, s);
  else if (M <= 8) launch_r<8, OT>(qt, w, a, y, M, N, K, s);
  else launch_r<16, OT>(qt, w, a, y, M, N, K, s);
}

int check_args(int qt, const void* w, void* y, int M, int N, int K, const char* nm) {
  UB_REQUIRE(qt == UB_Q4_0 || qt == UB_Q8_0 || qt == UB_Q4_K, "%s: unsupported qtype %d", nm, qt);
  UB_REQUIRE(w && y, "%s: null pointer", nm);
  UB_REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative shape", nm);
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
  UB_REQUIRE(workspace, "%s: null workspace", nm);
  UB_REQUIRE(y_dtype == UB_F32 || y_dtype == UB_BF16, "%s: y_dtype %d", nm, y_dtype);
  if (M == 0 || N == 0) return UB_OK;
  hipStream_t s = ub_stream(stream);
  for (int m0 = 0; m0 < M; m0 += 16) {
    int mc = M - m0 < 16 ? M - m0 : 16;
    ActWs a = carve(const_cast<void*>(workspace), qtype, M, K);
    a.q += (size_t)m0 * K;
    a.d += (size_t)m0 * K / (qtype == UB_Q4_K ? 256 : 32);
    a.s += (size_t)m0 * K / (qtype == UB_Q4_K ? 16 : 32);
    size_t yo = (size_t)m0 * N * (y_dtype == UB_F32 ? 4 : 2);
    void* yc = (uint8_t*)y + yo;
    if (K == 0) {
      size_t nbytes = (size_t)mc * N * (y_dtype == UB_F32 ? 4 : 2);
      k_zero<<<ub_cdiv((long)nbytes, 256) < 4096 ? ub_cdiv((long)nbytes, 256) : 4096, 256, 0, s>>>(
          (uint8_t*)yc, nbytes);
      continue;
    }
    if (y_dtype == UB_F32) launch_m<UB_F32>(qtype, (const uint8_t*)w, a, yc, mc, N, K, s);
    else launch_m<UB_BF16>(qtype, (const uint8_t*)w, a, yc, mc, N, K, s);
  }
  return ub_check_launch(nm);
}

// One-call form: quantize x then run the fused GEMV.
UB_API int ubridge_qmatmul(int qtype, const void* w, const void* x, int x_dtype, void* y,
                           int y_dtype, int M, int N, int K, void* workspace, size_t ws_bytes,
                           void* stream) {
  int e = ubridge_quantize_activations(qtype, x, x_dtype, M, K, workspace, ws_bytes, stream);
  if (e) return e;
  return ubridge_qmatmul_prequantized(qtype, w, y, y_dtype, M, N, K, workspace, stream);
}
