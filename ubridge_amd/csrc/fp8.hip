// fp8.hip -- fp8 (OCP e4m3fn) W8A8 GEMM on CDNA4 MFMA, gfx950.
//
//   out[m, n] = bf16( (sum_k a[m,k] * w[n,k]) * sa[m] * sw[n] )
//
// a: e4m3 [M, K] with per-token f32 scales sa [M]; w: e4m3 [N, K] (K
// contiguous, prepacked once from the [K, N] layout by ubridge_fp8_transpose)
// with per-output-channel f32 scales sw [N].  The reference has no fp8 path;
// the formula is the dense matmul of the decoded operands with the two scale
// vectors folded into the epilogue.
//
// Tiling: 128 x 128 block tile, 4 wavefronts (2 x 2) of 64 x 64, each a 2 x 2
// grid of v_mfma_scale_f32_32x32x64_f8f6f4 (block scale fixed at 2^0);
// BK = 128 bytes, double-buffered LDS with 16-byte row padding; global loads
// are raw buffer loads issued one K-step ahead.
#include "common.h"

namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kOOB = 0x80000000u;
constexpr int FBM = 128, FBN = 128, FBK = 128, FLD = FBK + 16;  // bytes

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint64_t bytes) {
  const uint32_t n = bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)n, 0x00020000);
}
__device__ __forceinline__ uint4 ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

__global__ void __launch_bounds__(256, 2) k_fp8_gemm(const uint8_t* __restrict__ A,
                                                     const float* __restrict__ sa,
                                                     const uint8_t* __restrict__ W,
                                                     const float* __restrict__ sw,
                                                     uint16_t* __restrict__ out, int M, int K,
                                                     int N) {
  __shared__ __align__(16) uint8_t As[2][FBM * FLD];
  __shared__ __align__(16) uint8_t Bs[2][FBN * FLD];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int n0 = blockIdx.x * FBN, m0 = blockIdx.y * FBM;
  const __amdgpu_buffer_rsrc_t ra = rsrc(A, (uint64_t)M * K);
  const __amdgpu_buffer_rsrc_t rw = rsrc(W, (uint64_t)N * K);
  // thread -> row tid/2, 64-byte half tid%2 of the 128-byte K-step
  const int row = tid >> 1, half = tid & 1;
  uint4 ar[4], br[4];
  auto load = [&](int k0) {
    const int k = k0 + 64 * half;
    const bool oka = m0 + row < M, okb = n0 + row < N;
    const uint32_t oa = (uint32_t)((size_t)(m0 + row) * K + k);
    const uint32_t ob = (uint32_t)((size_t)(n0 + row) * K + k);
#pragma unroll
    for (int i = 0; i < 4; i++) {  // K % 16 == 0: each 16-byte chunk is all in or all out
      const bool okk = k + 16 * i < K;
      ar[i] = ld16(ra, oka && okk ? oa + 16 * i : kOOB);
      br[i] = ld16(rw, okb && okk ? ob + 16 * i : kOOB);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      *(uint4*)(As[buf] + row * FLD + 64 * half + 16 * i) = ar[i];
      *(uint4*)(Bs[buf] + row * FLD + 64 * half + 16 * i) = br[i];
    }
  };
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;
  const int nk = (K + FBK - 1) / FBK;
  load(0);
  store(0);
  __syncthreads();
  const int l32 = lane & 31, kh = lane >> 5;
  for (int kt = 0; kt < nk; kt++) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) load((kt + 1) * FBK);
#pragma unroll
    for (int ks = 0; ks < FBK / 64; ks++) {
      i32x8 af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const uint8_t* p = As[cur] + (wm * 64 + 32 * i + l32) * FLD + 64 * ks + 32 * kh;
        const uint4 x0 = *(const uint4*)p, x1 = *(const uint4*)(p + 16);
        af[i] = (i32x8){(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w,
                        (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
        const uint8_t* q = Bs[cur] + (wn * 64 + 32 * i + l32) * FLD + 64 * ks + 32 * kh;
        const uint4 y0 = *(const uint4*)q, y1 = *(const uint4*)(q + 16);
        bfr[i] = (i32x8){(int)y0.x, (int)y0.y, (int)y0.z, (int)y0.w,
                         (int)y1.x, (int)y1.y, (int)y1.z, (int)y1.w};
      }
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[i], bfr[j], acc[i][j], 0,
                                                                      0, 0, 127, 0, 127);
    }
    if (more) store(cur ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int n = n0 + wn * 64 + 32 * j + l32;
      if (n >= N) continue;
      const float swn = sw[n];
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int m = m0 + wm * 64 + 32 * i + 8 * (r >> 2) + 4 * kh + (r & 3);
        if (m < M) {
          const float v = acc[i][j][r] * sa[m] * swn;
          out[(size_t)m * N + n] = __builtin_bit_cast(unsigned short, (__bf16)v);
        }
      }
    }
}

// [R, C] bytes -> [C, R] bytes through a 64 x 64 LDS tile.
__global__ void __launch_bounds__(256) k_transpose_u8(const uint8_t* __restrict__ in,
                                                      uint8_t* __restrict__ out, int R, int C) {
  __shared__ uint8_t tile[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int r = i / 64, c = i % 64;
    if (r0 + r < R && c0 + c < C) tile[r][c] = in[(size_t)(r0 + r) * C + c0 + c];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int c = i / 64, r = i % 64;
    if (r0 + r < R && c0 + c < C) out[(size_t)(c0 + c) * R + r0 + r] = tile[r][c];
  }
}

// Per-row fp8 quantization: scale = amax / 448 (1 for an all-zero row),
// q = e4m3(x / scale) with round-to-nearest-even (v_cvt_pk_fp8_f32).
template <int DT>
__global__ void __launch_bounds__(256) k_quant_rows_fp8(const void* __restrict__ x,
                                                        uint8_t* __restrict__ q,
                                                        float* __restrict__ scale, int R, int C) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;
  auto ld = [&](size_t i) -> float {
    if constexpr (DT == UB_F32) return ((const float*)x)[i];
    else if constexpr (DT == UB_F16) return ub_f16_to_f32(((const uint16_t*)x)[i]);
    else return ub_bf16_to_f32(((const uint16_t*)x)[i]);
  };
  float amax = 0.f;
  for (int c = lane; c < C; c += 64) amax = fmaxf(amax, fabsf(ld((size_t)r * C + c)));
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  const float s = amax > 0.f ? __fdiv_rn(amax, 448.0f) : 1.0f;
  for (int c = lane; c < C; c += 64) {
    const float v = __fdiv_rn(ld((size_t)r * C + c), s);
    const int pk = __builtin_amdgcn_cvt_pk_fp8_f32(v, v, 0, false);
    q[(size_t)r * C + c] = (uint8_t)(pk & 0xff);
  }
  if (lane == 0) scale[r] = s;
}

}  // namespace

// out[M,N] bf16 = (a[M,K] e4m3 . w[N,K]^T e4m3) * sa[M] (rows) * sw[N] (columns)
UB_API int ubridge_fp8_gemm(const uint8_t* a, const float* sa, const uint8_t* w_nk, const float* sw,
                            void* out, int M, int K, int N, void* stream) {
  const char* nm = "ubridge_fp8_gemm";
  UB_REQUIRE(M >= 0 && N >= 0 && K >= 0 && K % 16 == 0, "%s: M=%d K=%d (multiple of 16) N=%d", nm,
             M, K, N);
  if ((size_t)M * N == 0) return UB_OK;
  UB_REQUIRE(a && sa && w_nk && sw && out, "%s: null pointer", nm);
  dim3 grid(ub_cdiv(N, FBN), ub_cdiv(M, FBM));
  k_fp8_gemm<<<grid, 256, 0, ub_stream(stream)>>>(a, sa, w_nk, sw, (uint16_t*)out, M, K, N);
  return ub_check_launch(nm);
}

// Weight prepack: w_kn [K, N] -> w_nk [N, K] (bytes; done once at load time).
UB_API int ubridge_fp8_transpose(const uint8_t* in, uint8_t* out, int R, int C, void* stream) {
  UB_REQUIRE(R >= 0 && C >= 0, "ubridge_fp8_transpose: shape");
  if ((size_t)R * C == 0) return UB_OK;
  UB_REQUIRE(in && out && in != out, "ubridge_fp8_transpose: pointers");
  dim3 grid(ub_cdiv(C, 64), ub_cdiv(R, 64));
  k_transpose_u8<<<grid, 256, 0, ub_stream(stream)>>>(in, out, R, C);
  return ub_check_launch("ubridge_fp8_transpose");
}

// Per-row quantization of x [R, C] (f32 / f16 / bf16) to e4m3 + f32 row scales.
UB_API int ubridge_fp8_quantize_rows(const void* x, int x_dtype, uint8_t* q, float* scale, int R,
                                     int C, void* stream) {
  UB_REQUIRE(R >= 0 && C >= 0, "ubridge_fp8_quantize_rows: shape");
  if ((size_t)R * C == 0) return UB_OK;
  UB_REQUIRE(x && q && scale, "ubridge_fp8_quantize_rows: null pointer");
  hipStream_t s = ub_stream(stream);
  const int g = ub_cdiv(R, 4);
  if (x_dtype == UB_F32) k_quant_rows_fp8<UB_F32><<<g, 256, 0, s>>>(x, q, scale, R, C);
  else if (x_dtype == UB_F16) k_quant_rows_fp8<UB_F16><<<g, 256, 0, s>>>(x, q, scale, R, C);
  else k_quant_rows_fp8<UB_BF16><<<g, 256, 0, s>>>(x, q, scale, R, C);
  return ub_check_launch("ubridge_fp8_quantize_rows");
}
