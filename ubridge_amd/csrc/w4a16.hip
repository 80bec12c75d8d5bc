// w4a16.hip -- pipelined W4A16 GEMM for GPTQ-layout int4 weights (gfx950).
//
//   C[M, N] = A[M, K] . deq(W)[K, N],   deq(W)[k][n] = T((q[k][n] - z[g][n]) * s[g][n])
//
// A and C bf16 / f16, q int32 [K/8, N] (8 k-consecutive nibbles, LSB first),
// s T [K/g, N], z int32 [K/g, N/8] (8 n-consecutive nibbles), f32 accumulate:
// the same contract and rounding as the W_GPTQ4 producer of gemm.hip, which
// stays the fallback for group sizes or K that are not multiples of 64.
//
// Design (one workgroup of 8 wavefronts, 2 x 4, per BM x 256 tile, BK = 64):
//  * Every operand travels HBM -> LDS by direct-to-LDS buffer loads (no VGPR
//    staging), through a ring of 3 K-step stages, so two K-steps of loads are
//    in flight while the MFMAs consume the third (explicit vmcnt waits and
//    one barrier per K-step; the K loop is unrolled by 3 over the stages).
//  * The A tile is stored XOR-swizzled in 16-byte units (unit c of row r at
//    c ^ ((r >> 1) & 7)) so the 16 rows a fragment read touches per pass hit
//    distinct banks; the swizzle is applied on the global side of the load.
//  * The weight stays packed in LDS (8 KiB per stage instead of 32 KiB of
//    bf16) and is dequantized per MFMA fragment: one int32 word is exactly
//    the 8 k-consecutive values a lane feeds to v_mfma_f32_32x32x16 for its
//    column, so each lane turns one LDS word into its B operand in registers.
//  * Scales and zero points of the K-step's group ride along in the stage.
#include "common.h"
#include "lds_dma.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;
constexpr int kBN = 256;

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
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));  // v_cvt_pk_bf16_f32
  } else {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
  }
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

// One packed word (8 k of one column) -> the lane's B operand, k order kept:
// T((q - z) * s), computed as fma(q, s, -z*s), exact in f32 (q*s and z*s are
// exact), then rounded once to T.
template <int DT>
__device__ __forceinline__ uint4 dequant_word(uint32_t w, float s, float zs) {
  typedef unsigned char u8x4 __attribute__((ext_vector_type(4)));
  // nibbles 2b (lo) and 2b+1 (hi) in byte b.  The identity DPP move hides
  // the masks from the optimizer, which would otherwise extract each nibble
  // with its own bit-field op instead of converting bytes directly
  // (v_cvt_f32_ubyte0..3).
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(w & 0x0F0F0F0Fu), 0xE4, 0xf, 0xf, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)((w >> 4) & 0x0F0F0F0Fu), 0xE4, 0xf, 0xf, false);
  const u8x4 L = __builtin_bit_cast(u8x4, lo), H = __builtin_bit_cast(u8x4, hi);
  uint32_t o[4];
#pragma unroll
  for (int b = 0; b < 4; b++)
    o[b] = pack2<DT>(__builtin_fmaf((float)L[b], s, -zs), __builtin_fmaf((float)H[b], s, -zs));
  return make_uint4(o[0], o[1], o[2], o[3]);
}

struct W4Args {
  const void* a;
  const int32_t* qw;
  const void* scales;
  const int32_t* qzeros;
  void* c;
  int M, N, K, group;
};

// WM wavefronts along M x 4 along N (wave tile BM/WM x 64).  WM = 1 gives
// every weight fragment to one wave only (dequantized once per workgroup,
// reused by BM/32 MFMAs) at one wave per SIMD with up to 512 registers.
template <int DT, int BM, int WM>
__global__ void __launch_bounds__(256 * WM)
    __attribute__((amdgpu_waves_per_eu(WM, WM))) k_w4a16(W4Args p) {
  constexpr int kWaves = 4 * WM;
  constexpr int TM = BM / WM / 32;  // 32x32 tiles per wave along M
  constexpr int TN = kBN / 128;     // along N (wave tile 64 columns)
  constexpr int AB = BM * kBK * 2;  // A bytes per stage
  constexpr int WB = 8 * kBN * 4;   // packed-weight bytes per stage
  constexpr int SB = kBN * 2 + kBN / 2;  // scales + zero points per stage
  constexpr int NA = AB / (16 * 64 * kWaves);  // A load instructions per wave and stage
  constexpr int NL = NA + 8 / kWaves + 2;        // all load instructions per wave and stage
  // three stages, each one LDS object (A tile | packed weight | scales, zeros)
  __shared__ __attribute__((aligned(16))) uint8_t st0[AB + WB + SB], st1[AB + WB + SB],
      st2[AB + WB + SB];
  uint8_t *la0 = st0, *lw0 = st0 + AB, *ls0 = st0 + AB + WB;
  uint8_t *la1 = st1, *lw1 = st1 + AB, *ls1 = st1 + AB + WB;
  uint8_t *la2 = st2, *lw2 = st2 + AB, *ls2 = st2 + AB + WB;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;  // (wm = 0 when WM = 1)
  int tile_m, tile_n;
  ub_tile_order((p.M + BM - 1) / BM, (p.N + kBN - 1) / kBN, 8, tile_m, tile_n);
  const int n0 = tile_n * kBN, m0 = tile_m * BM;
  const int M = p.M, N = p.N, K = p.K;
  const ub_u32x4 ra = ub_desc(p.a, (uint64_t)M * K * 2);
  const ub_u32x4 rw = ub_desc(p.qw, (uint64_t)(K / 8) * N * 4);
  const int ng = K / p.group;
  const ub_u32x4 rs = ub_desc(p.scales, (uint64_t)ng * N * 2);
  const ub_u32x4 rz = ub_desc(p.qzeros, (uint64_t)ng * (N / 8) * 4);

  // ---- loads of K-step kt into one stage: per wave NA + 8 / kWaves + 2
  // instructions
  auto issue = [&](int kt, uint8_t* la, uint8_t* lw, uint8_t* ls) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < NA; i++) {
      const int u = (i * kWaves + wave) * 64 + lane;  // 16-byte unit of the stage
      const int row = u >> 3, c = (u & 7) ^ ((row >> 1) & 7);
      const int m = m0 + row;
      ub_lds_load16(ra, la + (i * kWaves + wave) * 1024,
                 m < M ? (uint32_t)(((size_t)m * K + k0) * 2 + c * 16) : kDmaOOB);
    }
#pragma unroll
    for (int i = 0; i < 8 / kWaves; i++) {  // packed weight: 8 word-rows x 256 columns (1 KiB)
      const int wr = i * kWaves + wave, n = n0 + 4 * lane;
      ub_lds_load16(rw, lw + wr * 1024,
                 n < N ? (uint32_t)(((size_t)(k0 / 8 + wr) * N + n) * 4) : kDmaOOB);
    }
    {  // scales: 32 units, zero points: 8 units, split evenly over the waves
      const int g = k0 / p.group;
      constexpr int SU = 32 / kWaves, ZU = 8 / kWaves;
      if (lane < SU) {
        const int n = n0 + 8 * (SU * wave + lane);
        ub_lds_load16(rs, ls + 16 * SU * wave, n < N ? (uint32_t)(((size_t)g * N + n) * 2) : kDmaOOB);
      }
      if (lane < ZU) {
        const int z8 = n0 / 8 + 4 * (ZU * wave + lane);
        ub_lds_load16(rz, ls + kBN * 2 + 16 * ZU * wave,
                   z8 < N / 8 ? (uint32_t)(((size_t)g * (N / 8) + z8) * 4) : kDmaOOB);
      }
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
  const int arow0 = wm * (BM / WM) + l32;
  const int ncol0 = wn * (kBN / 4) + l32;  // the lane's column in tile j: ncol0 + 32 j

  // ---- one K-step from one stage
  auto compute = [&](const uint8_t* la, const uint8_t* lw, const uint8_t* ls) {
    float sj[TN], zsj[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int n = ncol0 + 32 * j;
      sj[j] = tof<DT>(*(const uint16_t*)(ls + n * 2));
      const uint32_t zw = *(const uint32_t*)(ls + kBN * 2 + (n >> 3) * 4);
      zsj[j] = (float)((zw >> (4 * (n & 7))) & 15) * sj[j];
    }
    // fragments double-buffered across the four 16-k substeps: the LDS reads
    // of substep kk+1 are in flight while substep kk's dequant and MFMAs run
    uint4 af[2][TM];
    uint32_t bw[2][TN];
    auto load_frags = [&](int kk, int buf) {
      const int c = 2 * kk + kh;
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const int row = arow0 + 32 * i;
        af[buf][i] = *(const uint4*)(la + row * 128 + ((c ^ ((row >> 1) & 7)) * 16));
      }
#pragma unroll
      for (int j = 0; j < TN; j++)
        bw[buf][j] = *(const uint32_t*)(lw + ((2 * kk + kh) * kBN + ncol0 + 32 * j) * 4);
    };
    uint4 bfr[2][TN];
    load_frags(0, 0);
#pragma unroll
    for (int j = 0; j < TN; j++) bfr[0][j] = dequant_word<DT>(bw[0][j], sj[j], zsj[j]);
#pragma unroll
    for (int kk = 0; kk < kBK / 16; kk++) {
      const int cur = kk & 1, nxt = cur ^ 1;
      if (kk + 1 < kBK / 16) load_frags(kk + 1, nxt);
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = mfma<DT>(af[cur][i], bfr[cur][j], acc[i][j]);
      // next substep's B operands: VALU work that overlaps this substep's MFMAs
      if (kk + 1 < kBK / 16) {
#pragma unroll
        for (int j = 0; j < TN; j++) bfr[nxt][j] = dequant_word<DT>(bw[nxt][j], sj[j], zsj[j]);
      }
      // Interleave this substep's MFMAs with the next substep's LDS reads and
      // dequant VALU work: issue is in order, so VALU ops placed after a run
      // of MFMAs would wait for all of them to issue; spread between the
      // MFMAs they execute while the matrix pipe is busy.
#pragma unroll
      for (int q = 0; q < TM * TN; q++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        if (q < TM + TN) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 DS read
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // up to 3 VALU
      }
    }
  };

  // Per step: this wave's loads of the step are done (vmcnt: only the next
  // step's NL may be outstanding, or none at the last step), a barrier
  // makes every wave's loads visible and retires the previous step's reads,
  // then the loads of step + 2 go out into the stage read last step.
  const int nk = K / kBK;
  auto step = [&](int kt, uint8_t* la, uint8_t* lw, uint8_t* ls, uint8_t* la2_, uint8_t* lw2_,
                  uint8_t* ls2_) {
    if (kt + 1 < nk) ub_wait_vmcnt<NL>();
    else ub_wait_vmcnt<0>();
    ub_barrier();
    if (kt + 2 < nk) issue(kt + 2, la2_, lw2_, ls2_);
    compute(la, lw, ls);
  };

  issue(0, la0, lw0, ls0);
  if (nk > 1) issue(1, la1, lw1, ls1);
  for (int kt = 0; kt < nk; kt += 3) {
    step(kt, la0, lw0, ls0, la2, lw2, ls2);
    if (kt + 1 < nk) step(kt + 1, la1, lw1, ls1, la0, lw0, ls0);
    if (kt + 2 < nk) step(kt + 2, la2, lw2, ls2, la1, lw1, ls1);
  }

  // epilogue: lane l, register r of tile (i, j) holds
  // C[m0 + wm*BM/WM + 32i + 8(r/4) + 4(l/32) + r%4][n0 + wn*64 + 32j + l%32]
  uint16_t* C = (uint16_t*)p.c;
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int n = n0 + ncol0 + 32 * j;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int m = m0 + wm * (BM / WM) + 32 * i + 8 * (r >> 2) + 4 * kh + (r & 3);
        if (m < M && n < N) C[(size_t)m * N + n] = (uint16_t)(pack2<DT>(acc[i][j][r], 0.f) & 0xffff);
      }
    }
}

template <int DT, int BM>
int launch(const W4Args& a, hipStream_t s) {
  dim3 grid(ub_cdiv(a.N, kBN) * ub_cdiv(a.M, BM));
  if (ub_tune(UB_TUNE_W4A16_PATH) == 2) k_w4a16<DT, BM, 2><<<grid, 512, 0, s>>>(a);
  else k_w4a16<DT, BM, 1><<<grid, 256, 0, s>>>(a);
  return ub_check_launch("w4a16 gemm");
}

}  // namespace

// Pipelined W4A16 GEMM; returns UB_ERR_UNSUPPORTED (without recording an
// error) when the shape is outside its contract, so the caller can fall back.
int ub_w4a16_pipelined(const void* a, const int32_t* qw, const void* scales, const int32_t* qzeros,
                       void* out, int M, int K, int N, int group, int dtype, hipStream_t s) {
  if (group % kBK != 0 || K % kBK != 0 || K < kBK || N % 8 != 0) return UB_ERR_UNSUPPORTED;
  if ((uint64_t)M * K * 2 >= 0x80000000ull || (uint64_t)(K / 8) * N * 4 >= 0x80000000ull)
    return UB_ERR_UNSUPPORTED;  // 32-bit buffer offsets
  W4Args p{a, qw, scales, qzeros, out, M, N, K, group};
  // 256-row tiles once they fill the CUs, else 128
  const long tiles256 = (long)ub_cdiv(N, kBN) * ub_cdiv(M, 256);
  int t = ub_tune(UB_TUNE_GEMM_TILE);
  const bool big = t == 3 || (t == 0 && tiles256 >= 384);
  if (dtype == UB_BF16) return big ? launch<UB_BF16, 256>(p, s) : launch<UB_BF16, 128>(p, s);
  return big ? launch<UB_F16, 256>(p, s) : launch<UB_F16, 128>(p, s);
}
