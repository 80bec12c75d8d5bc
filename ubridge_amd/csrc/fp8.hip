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
// Tiling: 256 x 256 block tile, 8 wavefronts (2 along M x 4 along N, two per
// SIMD) of 128 x 64 (or 4 of 128 x 128, one per SIMD: knob gemm_tile 2), each
// a grid of v_mfma_scale_f32_32x32x64_f8f6f4 (block scale fixed at 2^0).
// Operands reach LDS by direct-to-LDS buffer loads in 64-byte K-steps, each
// 64-byte tile row XOR-swizzled in 16-byte units (unit c of row r at
// c ^ ((r >> 2) & 3)) so the 16 rows of a fragment read pass land in distinct
// banks.  k_fp8_gemm: a ring of 3 K-steps, one barrier per K-step;
// k_fp8_gemm2 (the default when K % 128 == 0): two stages of two K-steps, one
// barrier per 16 MFMAs per wavefront.  Fragments are read into registers one
// K-step ahead, between the MFMAs.
#include "common.h"
#include "lds_dma.h"

#include <type_traits>

int ub_blaslt_fp8(const uint8_t* a, const float* sa, const uint8_t* w_nk, const float* sw,
                  void* out, int M, int K, int N, hipStream_t s);

namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kOOB = 0x80000000u;
constexpr int FBM = 256, FBN = 256, FBK = 64;  // tile (K in bytes)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint64_t bytes) {
  const uint32_t n = bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)n, 0x00020000);
}
__device__ __forceinline__ uint4 ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// WN wavefronts along N (2 x WN wavefronts; wave tile 128 x 256/WN).
template <int WN>
__global__ void __launch_bounds__(128 * WN) __attribute__((amdgpu_waves_per_eu(WN / 2, WN / 2)))
k_fp8_gemm(const uint8_t* __restrict__ A, const float* __restrict__ sa,
           const uint8_t* __restrict__ W, const float* __restrict__ sw,
           uint16_t* __restrict__ out, int M, int K, int N) {
  constexpr int BM = FBM, BN = FBN, BK = FBK, TM = 4, TN = 8 / WN, NW = 2 * WN;
  constexpr int NI = 16 / NW;  // A (and B) load instructions per wave and stage
  constexpr int AB = BM * BK, STB = (BM + BN) * BK;  // bytes per stage
  __shared__ __attribute__((aligned(16))) uint8_t st0[STB], st1[STB], st2[STB];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  int tile_m, tile_n;
  ub_tile_order((M + BM - 1) / BM, (N + BN - 1) / BN, 8, tile_m, tile_n);
  const int n0 = tile_n * BN, m0 = tile_m * BM;
  const ub_u32x4 ra = ub_desc(A, (uint64_t)M * K);
  const ub_u32x4 rw = ub_desc(W, (uint64_t)N * K);

  // 16-byte unit u of a 256-row x 64-byte tile: row u/4, stored unit u%4
  // holds logical unit (u%4) ^ ((row >> 2) & 3).  NI + NI instructions per wave.
  auto issue = [&](int kt, uint8_t* st) {
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < NI; i++) {
      const int u = (i * NW + wave) * 64 + lane;
      const int row = u >> 2, c = (u & 3) ^ ((row >> 2) & 3);
      const int k = k0 + 16 * c;
      const int m = m0 + row, n = n0 + row;
      ub_lds_load16(ra, st + (i * NW + wave) * 1024,
                    m < M && k < K ? (uint32_t)((size_t)m * K + k) : kDmaOOB);
      ub_lds_load16(rw, st + AB + (i * NW + wave) * 1024,
                    n < N && k < K ? (uint32_t)((size_t)n * K + k) : kDmaOOB);
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  const int l32 = lane & 31, kh = lane >> 5;
  // lane's fragment: row l32 of the 32-row tile, bytes 32 kh .. +31 (units 2kh, 2kh+1)
  auto frag = [&](const uint8_t* t, int row) -> i32x8 {
    const int sw_ = (row >> 2) & 3;
    const uint4 x0 = *(const uint4*)(t + row * BK + (((2 * kh) ^ sw_) * 16));
    const uint4 x1 = *(const uint4*)(t + row * BK + (((2 * kh + 1) ^ sw_) * 16));
    return (i32x8){(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w,
                   (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
  };
  // Fragments live in registers, double-buffered by step parity, and are read
  // one step ahead: step kt starts its MFMAs on fragments read during step
  // kt-1, and while they run waits for stage kt+1, syncs, sends stage kt+3's
  // loads into the stage kt just vacated, and reads stage kt+1's fragments.
  i32x8 af[2][TM], bfr[2][TN];
  auto read_frags = [&](const uint8_t* st, int b) {
#pragma unroll
    for (int i = 0; i < TM; i++) af[b][i] = frag(st, wm * 128 + 32 * i + l32);
#pragma unroll
    for (int j = 0; j < TN; j++) bfr[b][j] = frag(st + AB, wn * (BN / WN) + 32 * j + l32);
  };
  const int nk = (K + BK - 1) / BK;
  uint8_t* stg[3] = {st0, st1, st2};
  // one step; S = kt % 3 (stage), B = kt % 2 (fragment buffer), both compile-time
  auto step = [&](auto Sc, auto Bc, int kt) {
    constexpr int S = decltype(Sc)::value, B = decltype(Bc)::value;
    // first MFMA column while the pipeline bookkeeping runs
#pragma unroll
    for (int i = 0; i < TM; i++)
      acc[i][0] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[B][i], bfr[B][0], acc[i][0],
                                                                  0, 0, 0, 127, 0, 127);
    if (kt + 1 < nk) {
      if (kt + 2 < nk) ub_wait_vmcnt<2 * NI>();  // stage kt+1 landed; kt+2 may be in flight
      else ub_wait_vmcnt<0>();
      ub_barrier();                                    // everyone is done reading stage kt
      if (kt + 3 < nk) issue(kt + 3, stg[S]);
      read_frags(stg[(S + 1) % 3], B ^ 1);
    }
#pragma unroll
    for (int j = 1; j < TN; j++)
#pragma unroll
      for (int i = 0; i < TM; i++)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[B][i], bfr[B][j], acc[i][j],
                                                                    0, 0, 0, 127, 0, 127);
    // spread the next step's fragment reads between the remaining MFMAs
#pragma unroll
    for (int q = 0; q < TM * (TN - 1); q++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // 2 DS reads
    }
  };
  issue(0, st0);
  if (nk > 1) issue(1, st1);
  if (nk > 2) issue(2, st2);
  if (nk > 2) ub_wait_vmcnt<4 * NI>();  // stage 0 landed (stages 1, 2 may be in flight)
  else if (nk > 1) ub_wait_vmcnt<2 * NI>();
  else ub_wait_vmcnt<0>();
  ub_barrier();
  read_frags(st0, 0);
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  for (int kt = 0; kt < nk; kt += 6) {
    step(I0{}, I0{}, kt);
    if (kt + 1 < nk) step(I1{}, I1{}, kt + 1);
    if (kt + 2 < nk) step(I2{}, I0{}, kt + 2);
    if (kt + 3 < nk) step(I0{}, I1{}, kt + 3);
    if (kt + 4 < nk) step(I1{}, I0{}, kt + 4);
    if (kt + 5 < nk) step(I2{}, I1{}, kt + 5);
  }
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int n = n0 + wn * (BN / WN) + 32 * j + l32;
      if (n >= N) continue;
      const float swn = sw[n];
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int m = m0 + wm * 128 + 32 * i + 8 * (r >> 2) + 4 * kh + (r & 3);
        if (m < M) {
          const float v = acc[i][j][r] * sa[m] * swn;
          out[(size_t)m * N + n] = __builtin_bit_cast(unsigned short, (__bf16)v);
        }
      }
    }
}

// The same tile with 128-byte K-steps: a stage is two 64-byte halves (each
// laid out as above) and the ring two stages, so a workgroup barrier comes
// every 16 MFMAs per wavefront instead of 8.  Step j: the MFMAs of half A
// run on fragments already in registers while half B's fragments are read;
// then stage j + 1 is waited for, the barrier frees stage j's buffers (its
// fragments are all in registers by then) for stage j + 2's loads, and the
// MFMAs of half B run while half A of stage j + 1 is read.  Loads are issued
// one step (16 MFMAs per wavefront) before they are waited for.
template <int WN>
__global__ void __launch_bounds__(128 * WN) __attribute__((amdgpu_waves_per_eu(WN / 2, WN / 2)))
k_fp8_gemm2(const uint8_t* __restrict__ A, const float* __restrict__ sa,
            const uint8_t* __restrict__ W, const float* __restrict__ sw,
            uint16_t* __restrict__ out, int M, int K, int N) {
  constexpr int BM = FBM, BN = FBN, BK = FBK, TM = 4, TN = 8 / WN, NW = 2 * WN;
  constexpr int NI = 16 / NW;
  constexpr int AB = BM * BK, STB = (BM + BN) * BK;  // bytes per half
  __shared__ __attribute__((aligned(16))) uint8_t h0[STB], h1[STB], h2[STB], h3[STB];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  int tile_m, tile_n;
  ub_tile_order((M + BM - 1) / BM, (N + BN - 1) / BN, 8, tile_m, tile_n);
  const int n0 = tile_n * BN, m0 = tile_m * BM;
  const ub_u32x4 ra = ub_desc(A, (uint64_t)M * K);
  const ub_u32x4 rw = ub_desc(W, (uint64_t)N * K);
  // half kt (64-byte K-step kt) into st (K % 128 == 0: every k is in range);
  // per-lane offsets set once, the step's as the scalar part
  uint32_t voA[NI], voW[NI];
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int u = (i * NW + wave) * 64 + lane;
    const int row = u >> 2, c = (u & 3) ^ ((row >> 2) & 3);
    const int m = m0 + row, n = n0 + row;
    voA[i] = m < M ? (uint32_t)((size_t)m * K + 16 * c) : kDmaOOB;
    voW[i] = n < N ? (uint32_t)((size_t)n * K + 16 * c) : kDmaOOB;
  }
  auto issue = [&](int kt, uint8_t* st) {
    const uint32_t sb = ub_lds_addr(st), k0 = (uint32_t)(kt * BK);
#pragma unroll
    for (int i = 0; i < NI; i++) {
      ub_lds_load16_at(ra, sb + (i * NW + wave) * 1024, voA[i], k0);
      ub_lds_load16_at(rw, sb + AB + (i * NW + wave) * 1024, voW[i], k0);
    }
  };
  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;
  const int l32 = lane & 31, kh = lane >> 5;
  auto frag = [&](const uint8_t* t, int row) -> i32x8 {
    const int sw_ = (row >> 2) & 3;
    const uint4 x0 = *(const uint4*)(t + row * BK + (((2 * kh) ^ sw_) * 16));
    const uint4 x1 = *(const uint4*)(t + row * BK + (((2 * kh + 1) ^ sw_) * 16));
    return (i32x8){(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w,
                   (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
  };
  i32x8 af[2][TM], bfr[2][TN];
  auto read_frags = [&](const uint8_t* st, int b) {
#pragma unroll
    for (int i = 0; i < TM; i++) af[b][i] = frag(st, wm * 128 + 32 * i + l32);
#pragma unroll
    for (int j = 0; j < TN; j++) bfr[b][j] = frag(st + AB, wn * (BN / WN) + 32 * j + l32);
  };
  auto mfmas = [&](int b) {
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int i = 0; i < TM; i++)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[b][i], bfr[b][j], acc[i][j],
                                                                    0, 0, 0, 127, 0, 127);
  };
  auto interleave = [&]() {
#pragma unroll
    for (int q = 0; q < TM * TN; q++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // 2 DS reads
    }
  };
  const int nks = K / (2 * BK);  // stages
  auto stage = [&](auto Pc, int j) {  // step j on buffer pair P = j % 2 (compile-time)
    constexpr int P = decltype(Pc)::value;
    uint8_t* a0 = P ? h2 : h0;
    uint8_t* a1 = P ? h3 : h1;
    uint8_t* n0b = P ? h0 : h2;  // next stage's half A
    // half A from registers; read half B
    mfmas(0);
    read_frags(a1, 1);
    interleave();
    if (j + 1 < nks) {
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this stage's fragment reads are done
      ub_wait_vmcnt<0>();                  // stage j + 1 landed (the only loads in flight)
      ub_barrier();                        // every wave is done reading stage j
      if (j + 2 < nks) {
        issue(2 * (j + 2), a0);
        issue(2 * (j + 2) + 1, a1);
      }
    }
    mfmas(1);
    read_frags(n0b, 0);  // (after the last stage: a harmless read of stale data)
    interleave();
  };
  issue(0, h0);
  issue(1, h1);
  if (nks > 1) {
    issue(2, h2);
    issue(3, h3);
    ub_wait_vmcnt<4 * NI>();  // stage 0 landed (stage 1 may be in flight)
  } else {
    ub_wait_vmcnt<0>();
  }
  ub_barrier();
  read_frags(h0, 0);
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  for (int j = 0; j < nks; j += 2) {
    stage(I0{}, j);
    if (j + 1 < nks) stage(I1{}, j + 1);
  }
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int n = n0 + wn * (BN / WN) + 32 * j + l32;
      if (n >= N) continue;
      const float swn = sw[n];
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int m = m0 + wm * 128 + 32 * i + 8 * (r >> 2) + 4 * kh + (r & 3);
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
  dim3 grid(ub_cdiv(N, FBN) * ub_cdiv(M, FBM));
  const int tile = ub_tune(UB_TUNE_GEMM_TILE);
  hipStream_t s = ub_stream(stream);
  // By default hipBLASLt's fp8 GEMM with per-row / per-column scale vectors
  // (configs[4] on MI355X: 753-757 against 882-888 us for the kernels below),
  // falling back to them when the library cannot serve the shape.  Knob
  // gemm_tile 3: the 128-byte K-step kernel below (one barrier per 16
  // MFMAs when K allows: 912 -> 883 us), 2: the 4-wavefront kernel, 4: the
  // 8-wavefront one with 64-byte K-steps.
  if (tile == 0 || tile == 1) {
    ub_blaslt_prepare(s);
    const int e = ub_blaslt_fp8(a, sa, w_nk, sw, out, M, K, N, s);
    if (e != UB_ERR_UNSUPPORTED) return e ? e : ub_check_launch(nm);
  }
  if (tile == 2)
    k_fp8_gemm<2><<<grid, 256, 0, s>>>(a, sa, w_nk, sw, (uint16_t*)out, M, K, N);
  else if (tile != 4 && K % 128 == 0)
    k_fp8_gemm2<4><<<grid, 512, 0, s>>>(a, sa, w_nk, sw, (uint16_t*)out, M, K, N);
  else
    k_fp8_gemm<4><<<grid, 512, 0, s>>>(a, sa, w_nk, sw, (uint16_t*)out, M, K, N);
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
