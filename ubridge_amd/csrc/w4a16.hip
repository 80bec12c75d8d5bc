// w4a16.hip -- pipelined W4A16 GEMM for GPTQ-layout int4 weights (gfx950).
//
//   C[M, N] = A[M, K] . deq(W)[K, N],   deq(W)[k][n] = T((q[k][n] - z[g][n]) * s[g][n])
//
// A and C bf16 / f16, q int32 [K/8, N] (8 k-consecutive nibbles, LSB first),
// s T [K/g, N], z int32 [K/g, N/8] (8 n-consecutive nibbles), f32 accumulate:
// the same contract and rounding as the W_GPTQ4 producer of gemm.hip, which
// stays the fallback for group sizes or K that are not multiples of 64.
//
// Design.  One workgroup of 8 wavefronts (two per SIMD, so one can issue
// while the other waits on LDS or a barrier) owns a BM x 256 output tile;
// each wavefront computes 128 x 64 of it with v_mfma_f32_32x32x16 (4 x 2
// MFMA tiles, 128 accumulators in AGPRs).  The wavefronts are 4 along N
// times either 2 along M (BM = 256) or 2 along K (BM = 128: each half of K
// is reduced through LDS at the end), so small-M problems still put one tile
// on every CU.  (A 4-wavefront variant with 128 x 128 wave tiles, one per
// SIMD, is kept behind the w4a16_path = 3 knob; it measured slower.  A
// variant whose 8 wavefronts each own 256 x 64 (TMX = 8: half the LDS B-reads
// and dequant VALU per MFMA) is behind w4a16_path = 5; it measured level.)  The
// 32 x 32 x 16 MFMA runs at full rate from one wavefront per SIMD, whereas
// the 16 x 16 x 32 bf16 form measured at half rate on gfx950.
//  * Every operand travels HBM -> LDS by direct-to-LDS buffer loads through a
//    ring of 3 K-step stages (BK = 64).  Per-lane global offsets are set up
//    once; each K-step adds a scalar offset.
//  * The A tile is XOR-swizzled in 16-byte units (unit c of row r at
//    c ^ ((r >> 1) & 7)); packed-weight rows are padded to 1152 bytes, so
//    both fragment reads are free of bank conflicts.
//  * The weight stays packed in LDS.  One int32 word is exactly the 8
//    k-consecutive values a lane feeds to the MFMA for its column, so each
//    lane turns one LDS word into its B operand in registers:
//    T((q - z) * s) = round(fma(q, s, -z s)), exact before the one rounding.
//  * Software pipeline over the 4 16-k substeps of a K-step: LDS reads run two
//    substeps ahead, the dequantization one substep ahead, and both are
//    interleaved between the MFMAs of the current substep.  The one barrier
//    per K-step sits between substeps 1 and 2: after it the next stage is
//    visible (its fragments are read from substep 2 on) and the current stage
//    is free (its last fragments were read in substep 1), so its buffer takes
//    the loads of the step three ahead and every stage has two K-steps to
//    arrive.
#include "common.h"
#include "lds_dma.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned char u8x4 __attribute__((ext_vector_type(4)));

constexpr int kBN = 256;
constexpr int kWRow = 1152;  // LDS bytes per packed-weight word-row (1024 used)

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

// One packed word (8 k of one column, LSB first) -> the lane's B operand,
// k order kept.  Low nibbles convert directly (v_cvt_f32_ubyteN); high
// nibbles are converted as 16 q and scaled by s/16, which is exact, so no
// shifts are needed: 2 masks + 8 converts + 8 fma + 4 packs.  The masks come
// in as registers the optimizer cannot see through (m_lo = 0x0f0f0f0f,
// m_hi = 0xf0f0f0f0), so it keeps the byte converts instead of rewriting
// them into bit-field extracts.
template <int DT>
__device__ __forceinline__ uint4 dequant_word(uint32_t w, uint32_t m_lo, uint32_t m_hi, float s,
                                              float s16, float zs) {
  const u8x4 L = __builtin_bit_cast(u8x4, w & m_lo), H = __builtin_bit_cast(u8x4, w & m_hi);
  uint32_t o[4];
#pragma unroll
  for (int b = 0; b < 4; b++)
    o[b] = pack2<DT>(__builtin_fmaf((float)L[b], s, -zs), __builtin_fmaf((float)H[b], s16, -zs));
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// Q4_K block header h (d, dmin as fp16 in h.x; scales[12] in h.y..h.w):
// the multipliers of the 64-k group GQ (sub-blocks 2 GQ, 2 GQ + 1) with the
// byte positions fixed at compile time: lo = d sc(2 GQ), zl = dmin m(2 GQ),
// hi16 = d sc(2 GQ + 1) / 16, zh = dmin m(2 GQ + 1), all exact in f32.
template <int GQ>
__device__ __forceinline__ void q4k_group(const uint4& h, float& lo, float& zl, float& hi16,
                                          float& zh) {
  const float d = ub_f16_to_f32((uint16_t)(h.x & 0xffff));
  const float dm = ub_f16_to_f32((uint16_t)(h.x >> 16));
  int c0, m0, c1, m1;
  q4k_scale_min(2 * GQ, h.y, h.z, h.w, c0, m0);
  q4k_scale_min(2 * GQ + 1, h.y, h.z, h.w, c1, m1);
  lo = d * (float)c0;
  zl = dm * (float)m0;
  hi16 = d * (float)c1 * 0.0625f;
  zh = dm * (float)m1;
}

// Weight formats (the W_* numbering of gemm.hip):
//   kGptq  int32 [K/8, N]: 8 k-consecutive nibbles, LSB first; zero points
//          int32 [K/g, N/8] (8 n-consecutive nibbles): T((q - z) s)
//   kU4    uint8 [K/2, N] (low nibble = even k); zeros T [K/g, N]:
//          T((q - z) s) with the subtraction rounded in f32 first
//   kI8Kn  int8 [K, N];  kI8Nk  int8 [N, K]: T(q s)
// Scales are T [K/g, N] in these formats.
//   kQ4K   GGUF Q4_K SoA weight [N, K] (qw: the 128-byte code payloads, qzeros:
//          the 16-byte headers d, dmin, scales[12]; block b = n K/256 + k/256):
//          bf16(d sc q - dmin m), the values of dequantize_block_q4_k_bf16.
//   kQ8_0  GGUF Q8_0 SoA [N, K] (qw: the 32-byte int8 payloads, i.e. int8
//          [N, K] row-major; qzeros: the fp16 scales d): bf16(bf16(d) q)
//   kQ4_0  GGUF Q4_0 SoA [N, K] (qw: 16-byte payloads, element e < 16 the low
//          nibble of byte e, e >= 16 the high nibble of byte e - 16; qzeros:
//          the fp16 scales d): bf16((q - 8) d)
// (the dequantize_block_*_bf16 values; the GGUF formats take bf16 only)
enum { kGptq = 0, kU4 = 1, kI8Kn = 2, kI8Nk = 3, kQ4K = 4, kQ8_0 = 5, kQ4_0 = 6 };
// GGUF formats: per-column header bytes of a 256-k span (Q4_K: its block
// header; Q8_0 / Q4_0: the 8 fp16 scales of its 32-k blocks) are 16 bytes,
// kept outside the ring.  kNib32: 32 code bytes per column and K-step (Q4_K,
// Q4_0); kNk64: 64 (int8 [N, K] and Q8_0).
constexpr bool kGguf(int wf) { return wf >= kQ4K; }
constexpr bool kNib32(int wf) { return wf == kQ4K || wf == kQ4_0; }
constexpr bool kNk64(int wf) { return wf == kI8Nk || wf == kQ8_0; }

struct W4Args {
  const void* a;
  const void* qw;
  const void* scales;
  const void* qzeros;
  void* c;
  int M, N, K, group;
  int c_f32;    // C is f32 (else T)
  int ksplit;   // > 1: workgroup (tile, blockIdx.y) takes K-steps [y, y + 1) K / 64 / ksplit
  float* part;  // and stores its f32 partial sums to part[y][M][N] (summed by k_ksum)
};

// LDS image of one K-step (64 k) of the weight for 256 columns.
//  kGptq: 8 word-rows (8 k each) of 256 x 4 bytes, rows padded to kWRow.
//  kU4 / kI8Kn: 16-byte units of 4 byte-rows x 4 columns, 64 units (256
//    columns) per unit-row; 8 unit-rows (kU4: 8 k each) or 16 (kI8Kn: 4 k
//    each).  Loaded by 4-byte direct-to-LDS loads whose lanes gather the
//    unit (4 byte-rows touched in 64-byte runs per instruction).
//  kI8Nk: 16 blocks of 16 columns x 64 k (1 KiB); 16-byte chunk c of column
//    n (n < 16 in the block) sits at unit 8 (n / 2) + ((4 (n & 1) + c) ^
//    (n / 2 & 7)), so the 8 lanes of one LDS read cycle (even columns, one
//    chunk) hit 8 different bank groups.
//  kQ4K: a column's 32 code bytes of the K-step (k < 32 the low nibbles of
//    bytes k, k >= 32 the high nibbles of bytes k - 32) as two 16-byte
//    halves; 8 blocks of 32 columns (1 KiB), half h of column c (c < 32 in
//    the block) at unit 32 h + 16 (c & 1) + c / 2, so the 16 lanes that read
//    one half of 16 even (or odd) columns read 256 contiguous bytes.  Loaded
//    by 16-byte direct-to-LDS loads, one block (32 columns x 32 bytes) per
//    instruction.  The 16-byte block headers serve 4 K-steps: they sit
//    outside the ring, two slots (256-k block parity) x KS halves x 256
//    columns, loaded with the first K-step of their block (or of the K-half).
template <int WF>
struct WGeo {
  static constexpr int WB = WF == kGptq ? 8 * kWRow : WF == kU4 || kNib32(WF) ? 8192 : 16384;
  static constexpr int SB = WF == kGptq ? kBN * 2 + kBN / 2
                            : WF == kU4 ? kBN * 4
                            : kGguf(WF) ? 0 : kBN * 2;
  static constexpr int WI = WF == kGptq || kNib32(WF) ? 8 : WF == kU4 ? 32 : WF == kI8Kn ? 64 : 16;  // loads per K-half
  static constexpr int RAW = WF == kGptq || WF == kU4 || kNib32(WF) ? 4 : 8;  // raw B words per lane and substep
};

// Block (32 TMX WM) x 256 with NV wavefronts: NV / (WM KS) along N x (WM
// along M, KS along K).  TMX = 4 (128-row wave tiles): WM KS = 2; NV = 4:
// one wavefront per SIMD, 128 x 128 each; NV = 8: two per SIMD, 128 x 64
// each; TMX = 2 (64-row wave tiles, for at most 64 rows): the same with 64
// x 64.  TMX = 8: WM = KS = 1, NV = 4, one wavefront per SIMD of 256 x 64:
// each dequantized weight fragment then feeds 8 MFMAs instead of 4.  NSTG
// K-step stages in the LDS ring (3, or 2 where 3 do not fit).
template <int WF, int DT, int WM, int KS, int NV, int TMX = 4, int NSTG = 3>
__global__ void __launch_bounds__(64 * NV) __attribute__((amdgpu_waves_per_eu(NV / 4, NV / 4)))
    k_w4a16(W4Args p) {
  static_assert(((TMX == 4 || TMX == 2) && WM * KS == 2) || (TMX == 8 && WM == 1 && KS == 1 && NV == 4),
                "wavefront layout");
  static_assert(NV == 4 || NV == 8, "4 or 8 wavefronts");
  static_assert(NSTG == 2 || NSTG == 3, "ring depth");
  static_assert(!kGguf(WF) || (NV == 8 && TMX <= 4 && DT == UB_BF16), "GGUF: 128 / 64 x 64 wave tiles, bf16");
  using G = WGeo<WF>;
  constexpr int WR = 32 * TMX;                // rows per wavefront tile
  constexpr int BM = WR * WM;
  constexpr int NWN = NV / (WM * KS);         // wavefronts along N
  constexpr int TM = TMX, TN = 8 / NWN;       // 32 x 32 MFMA tiles per wavefront
  constexpr int CW = 32 * TN;                 // columns per wavefront
  constexpr int AB = BM * 128;                // A bytes per half-stage: BM rows x 64 k
  constexpr int WB = G::WB;
  constexpr int SB = G::SB;                   // scales (+ zero points) of the K-step's group
  constexpr int HB = AB + WB + SB;            // one K-half of a stage
  constexpr int STB = KS * HB;                // stage
  constexpr int NA = KS * AB / 1024 / NV;     // A load instructions per wave and stage
  constexpr int NW = KS * G::WI / NV;         // weight load instructions per wave and stage
  // scale / zero-point loads per stage; kQ4K's header load (one stage in 4)
  // is left out of the count, which only makes the waits below stricter
  constexpr int NS = kGguf(WF) ? 0 : KS;
  constexpr int NL = NA + NW + NS;
  static_assert(KS * G::WI % NV == 0, "weight loads split evenly");
  constexpr int XB = KS == 2 ? TM * TN * 4096 * NWN : 0;  // split-K exchange
  constexpr int HR = NSTG * STB;                           // kQ4K header slots
  constexpr int RING = HR + (kGguf(WF) ? 2 * KS * kBN * 16 : 0);
  constexpr int SMEM = RING > XB ? RING : XB;
  static_assert(SMEM <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave % NWN;
  const int kh = KS == 2 ? wave / NWN : 0;
  const int wm = WM == 2 ? wave / NWN : 0;
  int tile_m, tile_n;
  ub_tile_order((p.M + BM - 1) / BM, (p.N + kBN - 1) / kBN, 8, tile_m, tile_n);
  const int n0 = tile_n * kBN, m0 = tile_m * BM;
  const int M = p.M, N = p.N, K = p.K;
  const int S = p.ksplit > 1 ? p.ksplit : 1;
  const int nkh = K / 64 / S / KS;             // K-steps per K-half
  const int kb = blockIdx.y * (K / 64 / S);    // first K-step of this workgroup
  const ub_u32x4 ra = ub_desc(p.a, (uint64_t)M * K * 2);
  const uint64_t wbytes = WF == kGptq ? (uint64_t)(K / 8) * N * 4
                          : WF == kU4 || kNib32(WF) ? (uint64_t)(K / 2) * N
                                      : (uint64_t)K * N;
  const ub_u32x4 rw = ub_desc(p.qw, wbytes);
  const int ng = K / p.group;
  const ub_u32x4 rs = ub_desc(p.scales, kGguf(WF) ? 0 : (uint64_t)ng * N * 2);
  const ub_u32x4 rz = ub_desc(p.qzeros, WF == kGptq ? (uint64_t)ng * (N / 8) * 4
                                        : WF == kU4 ? (uint64_t)ng * N * 2
                                        : kGguf(WF) ? (uint64_t)(K / 256) * N * 16 : 0);
  const uint32_t sbase = ub_lds_addr(smem);

  // ---- this wave's load instructions: per-lane offsets of K-step 0
  uint32_t voA[NA], voW[NW], voS;
#pragma unroll
  for (int i = 0; i < NA; i++) {
    const int U = (i * NV + wave) * 64;  // first 16-byte unit of the instruction
    const int h = U / (AB / 16), u = U % (AB / 16) + lane;
    const int row = u >> 3, c = (u & 7) ^ ((row >> 1) & 7);
    const int m = m0 + row;
    voA[i] = m < M ? (uint32_t)(((size_t)m * K + (kb + h * nkh) * 64 + 8 * c) * 2) : kDmaOOB;
  }
  // weight instruction j of this wave: R = j NV + wave of the stage's KS WI
  // instructions; lds_w[j] its LDS offset inside the stage
  uint32_t lds_w[NW];
#pragma unroll
  for (int j = 0; j < NW; j++) {
    const int R = j * NV + wave, h = R / G::WI, q = R % G::WI;
    if constexpr (WF == kGptq) {
      const int n = n0 + 4 * lane;
      voW[j] = n < N ? (uint32_t)(((size_t)((kb + h * nkh) * 8 + q) * N + n) * 4) : kDmaOOB;
      lds_w[j] = h * HB + AB + q * kWRow;
    } else if constexpr (WF == kU4 || WF == kI8Kn) {
      // unit-row q / 4, columns 64 (q % 4) + 4 (lane / 4), byte-row lane % 4
      constexpr int KR = WF == kU4 ? 32 : 64;  // byte-rows per K-step
      const int ur = q >> 2, n = n0 + 64 * (q & 3) + 4 * (lane >> 2);
      const int row = (kb + h * nkh) * KR + 4 * ur + (lane & 3);
      voW[j] = n < N ? (uint32_t)((size_t)row * N + n) : kDmaOOB;
      lds_w[j] = h * HB + AB + ur * 1024 + (q & 3) * 256;
    } else if constexpr (kNib32(WF)) {
      // block q; unit `lane` holds half lane / 32 of column 2 (lane % 16) +
      // (lane / 16) % 2 of the block (a column's codes: K / 2 bytes)
      const int hh = lane >> 5, n = n0 + 32 * q + 2 * (lane & 15) + ((lane >> 4) & 1);
      voW[j] = n < N ? (uint32_t)((size_t)n * (K / 2) + (kb + h * nkh) * 32 + 16 * hh) : kDmaOOB;
      lds_w[j] = h * HB + AB + q * 1024;
    } else {  // kI8Nk / kQ8_0: block q of 16 columns, unit `lane` of the block
      const int t = lane >> 3, low = (lane & 7) ^ (t & 7);
      const int n = n0 + 16 * q + 2 * t + (low >> 2), c = low & 3;
      voW[j] = n < N ? (uint32_t)((size_t)n * K + (kb + h * nkh) * 64 + 16 * c) : kDmaOOB;
      lds_w[j] = h * HB + AB + q * 1024;
    }
  }
  // scales: 32 16-byte units; zero points: 8 (kGptq) or 32 (kU4) units.
  // kGptq / kU4: the first half of the waves load scales, the second half
  // zero points; kI8*: every wave loads scales.
  constexpr int NSW = WF == kI8Kn || WF == kI8Nk ? NV : NV / 2;  // waves loading scales
  constexpr int SL = 32 / NSW, ZL = (WF == kU4 ? 32 : 8) / (NV / 2);  // units per wave
  const bool s_scale = wave < NSW;
  const int sidx = s_scale ? wave : wave - NSW;
  const bool s_on = s_scale ? lane < SL : lane < ZL;
  {
    const int n = n0 + 8 * (sidx * SL + lane);
    if (s_scale) voS = n < N ? (uint32_t)(n * 2) : kDmaOOB;
    else if constexpr (WF == kGptq) {
      const int z8 = n0 / 8 + 4 * (sidx * ZL + lane);
      voS = z8 < N / 8 ? (uint32_t)(z8 * 4) : kDmaOOB;
    } else {
      const int nz = n0 + 8 * (sidx * ZL + lane);
      voS = nz < N ? (uint32_t)(nz * 2) : kDmaOOB;
    }
  }
  uint32_t s_lds = AB + WB + (s_scale ? sidx * SL * 16 : kBN * 2 + sidx * ZL * 16);
  // kQ4K: every wave loads 32 KS headers, unit u = 32 KS wave + lane: K-half
  // u / 256, column u % 256
  const int hq_u = 32 * KS * wave + lane, hq_h = KS == 2 ? wave / 4 : 0;
  const bool hq_on = lane < 32 * KS;
  if constexpr (kGguf(WF)) {
    const int n = n0 + hq_u % kBN;
    voS = n < N ? (uint32_t)((size_t)n * (K / 256) * 16) : kDmaOOB;
    s_lds = HR + hq_h * kBN * 16 + (hq_u % kBN - lane) * 16;
  }

  auto issue = [&](int kt, uint32_t st) {
#pragma unroll
    for (int i = 0; i < NA; i++) {
      const int U = (i * NV + wave) * 64;
      const int h = U / (AB / 16), u0 = U % (AB / 16);
      ub_lds_load16_at(ra, st + h * HB + u0 * 16, voA[i], (uint32_t)kt * 128u);
    }
#pragma unroll
    for (int j = 0; j < NW; j++) {
      if constexpr (WF == kGptq)
        ub_lds_load16_at(rw, st + lds_w[j], voW[j], (uint32_t)kt * 32u * (uint32_t)N);
      else if constexpr (WF == kU4)
        ub_lds_load4_at(rw, st + lds_w[j], voW[j], (uint32_t)kt * 32u * (uint32_t)N);
      else if constexpr (WF == kI8Kn)
        ub_lds_load4_at(rw, st + lds_w[j], voW[j], (uint32_t)kt * 64u * (uint32_t)N);
      else if constexpr (kNib32(WF))
        ub_lds_load16_at(rw, st + lds_w[j], voW[j], (uint32_t)kt * 32u);
      else
        ub_lds_load16_at(rw, st + lds_w[j], voW[j], (uint32_t)kt * 64u);
    }
    if constexpr (kGguf(WF)) {
      const int ka = kt + kb + hq_h * nkh;  // wave-uniform
      // the first K-step of a block, or of the K-half (which may start inside one)
      if (((ka & 3) == 0 || kt == 0) && hq_on)
        ub_lds_load16_at(rz, sbase + s_lds + ((ka >> 2) & 1) * (KS * kBN * 16), voS,
                         (uint32_t)(ka >> 2) * 16u);
      return;
    }
#pragma unroll
    for (int h = 0; h < KS; h++) {
      const int g = (kt + kb + h * nkh) * 64 / p.group;
      if (s_on) {
        if (s_scale) ub_lds_load16_at(rs, st + h * HB + s_lds, voS, (uint32_t)(g * N * 2));
        else if constexpr (WF == kGptq)
          ub_lds_load16_at(rz, st + h * HB + s_lds, voS, (uint32_t)(g * (N / 8) * 4));
        else if constexpr (WF == kU4)
          ub_lds_load16_at(rz, st + h * HB + s_lds, voS, (uint32_t)(g * N * 2));
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

  // ---- fragment addressing (inside one K-half of a stage)
  const int l32 = lane & 31, kq = lane >> 5;
  const int sw = (l32 >> 1) & 7;
  // MFMA column slot l32 of tile j is physical column ncl + j: a lane's TN
  // columns are adjacent, so its scales and zero points are one LDS read
  // and its outputs one store per row.
  const int ncl = wn * CW + TN * l32;
  // A: row wm*128 + 32 i + l32, 16-byte chunk ck(s) of the 64-k row.  The
  // lane's 8 k of substep s are chunk 2 s + kq; for kI8Nk the k of a
  // substep pair are permuted (chunk 4 (s / 2) + 2 kq + s % 2, the same on
  // both operands) so that one column's 16 contiguous k bytes serve it.
  uint32_t aoff[4];
#pragma unroll
  for (int s = 0; s < 4; s++) {
    // kQ4_0: lane kq's 16 code bytes are 32-k block kq of the K-step, its
    // substeps the low (s < 2) then high nibbles of bytes 8 (s % 2) on:
    // chunk 4 kq + s
    const int ck = WF == kQ4_0 ? 4 * kq + s
                   : kNk64(WF) || WF == kQ4K ? 4 * (s >> 1) + 2 * kq + (s & 1) : 2 * s + kq;
    aoff[s] = (wm * WR + l32) * 128 + ((ck ^ sw) << 4);
  }
  // B: LDS offset of the lane's raw words of substep 0 of a K-half
  //  kGptq: word-row kq (+ 2 per substep); kU4: unit-row kq (+ 2 per
  //  substep); kI8Kn: unit-rows 2 kq, + 1 (+ 4 per substep); kI8Nk: the
  //  lane's columns, chunk kq (substeps 2, 3: chunk 2 + kq), 8 bytes per
  //  substep (s % 2).
  const uint32_t hoff = kh * HB;
  uint32_t boff = 0;
  if constexpr (WF == kGptq) boff = AB + kq * kWRow + ncl * 4;
  else if constexpr (WF == kU4) boff = AB + kq * 1024 + (ncl >> 2) * 16;
  else if constexpr (WF == kI8Kn) boff = AB + 2 * kq * 1024 + (ncl >> 2) * 16;
  // kQ4K / kQ4_0: unit of column nl (in the tile), half kq; the lane's
  // substep s reads bytes 8 (s % 2) of it, low nibbles in substeps 0, 1 and
  // high nibbles in 2, 3.  kQ4K: k = 16 kq + 8 (s % 2) + i (+ 32 for the high
  // nibbles), the kI8Nk k order; kQ4_0 (half kq = 32-k block kq): k = 32 kq
  // + 8 s + i.
  auto q4k_unit = [&](int nl) -> uint32_t {
    const int c = nl & 31;
    return AB + (nl >> 5) * 1024 + 16 * (32 * kq + 16 * (c & 1) + (c >> 1));
  };
  uint32_t bq4[TN];
#pragma unroll
  for (int j = 0; j < TN; j++) bq4[j] = kNib32(WF) ? q4k_unit(ncl + j) : 0;
  // kI8Nk: unit of column nl (in the tile), chunk c
  auto i8nk_unit = [&](int nl, int c) -> uint32_t {
    const int nb = nl & 15, t = nb >> 1;
    return AB + (nl >> 4) * 1024 + 16 * (8 * t + ((((nb & 1) << 2) | c) ^ (t & 7)));
  };
  uint32_t bnk[TN][2];  // kI8Nk: [column][substep pair]
#pragma unroll
  for (int j = 0; j < TN; j++)
#pragma unroll
    for (int pr = 0; pr < 2; pr++) bnk[j][pr] = kNk64(WF) ? i8nk_unit(ncl + j, 2 * pr + kq) : 0;
  // TN = 2 lanes of the 4-column units (kU4, kI8Kn) use columns (ncl & 3) + j
  const uint32_t bsh = (ncl & 2) ? 16u : 0u;

  uint4 af[4][TM];
  uint32_t bw[2][G::RAW];  // raw weight words of the lane's columns
  uint4 bf[2][TN];
  float sc[2][TN], s16[2][TN], zs[2][TN];  // [0]: this K-step, [1]: the next
  float zh[2][TN];                          // kQ4K: dmin m of the upper sub-block

  auto read_a = [&](uint32_t st, int s, int buf) {
#pragma unroll
    for (int i = 0; i < TM; i++) af[buf][i] = ub_lds_read16(st + hoff + aoff[s] + 4096 * i);
  };
  auto put4 = [&](int buf, int at, const uint4& v) {
    bw[buf][at] = v.x; bw[buf][at + 1] = v.y; bw[buf][at + 2] = v.z; bw[buf][at + 3] = v.w;
  };
  auto read_b = [&](uint32_t st, int s, int buf) {
    const uint32_t B = st + hoff;
    if constexpr (WF == kGptq) {
      if constexpr (TN == 4) {
        put4(buf, 0, ub_lds_read16(B + boff + 2 * s * kWRow));
      } else {
        const uint2 v = ub_lds_read8(B + boff + 2 * s * kWRow);
        bw[buf][0] = v.x; bw[buf][1] = v.y;
      }
    } else if constexpr (WF == kU4) {
      put4(buf, 0, ub_lds_read16(B + boff + 2 * s * 1024));
    } else if constexpr (kNib32(WF)) {
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const uint2 v = ub_lds_read8(B + bq4[j] + 8 * (s & 1));
        bw[buf][2 * j] = v.x; bw[buf][2 * j + 1] = v.y;
      }
    } else if constexpr (WF == kI8Kn) {
      put4(buf, 0, ub_lds_read16(B + boff + 4 * s * 1024));
      put4(buf, 4, ub_lds_read16(B + boff + 4 * s * 1024 + 1024));
    } else {
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const uint2 v = ub_lds_read8(B + bnk[j][s >> 1] + 8 * (s & 1));
        bw[buf][2 * j] = v.x; bw[buf][2 * j + 1] = v.y;
      }
    }
  };
  // scales / zero points of the next K-step: read raw in one substep,
  // converted in the next (after the reads have landed)
  uint2 s_raw, zt_raw;
  uint32_t z_raw;
  uint4 hq_raw[TN];  // kQ4K: block headers of the lane's columns
  // (kt: the K-step in this wave's K-half, for kQ4K's header slot)
  auto read_scales = [&](uint32_t st, int kt) {
    const uint32_t S = st + hoff + AB + WB;
    if constexpr (kGguf(WF)) {
      const uint32_t H =
          sbase + HR + ((((kt + kb + kh * nkh) >> 2) & 1) * KS + kh) * (kBN * 16) + ncl * 16;
#pragma unroll
      for (int j = 0; j < TN; j++) hq_raw[j] = ub_lds_read16(H + j * 16);
      return;
    }
    if constexpr (TN == 4) s_raw = ub_lds_read8(S + ncl * 2);
    else s_raw = make_uint2(ub_lds_read4(S + ncl * 2), 0);
    if constexpr (WF == kGptq) {
      z_raw = ub_lds_read4(S + kBN * 2 + (ncl >> 3) * 4);
    } else if constexpr (WF == kU4) {
      if constexpr (TN == 4) zt_raw = ub_lds_read8(S + kBN * 2 + ncl * 2);
      else zt_raw = make_uint2(ub_lds_read4(S + kBN * 2 + ncl * 2), 0);
    }
  };
  // per column: kGptq and kU4 sc = s, s16 = s / 16, zs = z s;
  // kI8* sc = s, zs = 128 s
  // kQ4K (gq: the K-step's 64-k group of its 256-k block, sub-blocks 2 gq
  // and 2 gq + 1): sc = d sc_lo, zs = dmin m_lo, s16 = d sc_hi / 16, zh =
  // dmin m_hi -- d sc and dmin m exact in f32
  // kQ8_0: sc = d of the K-step's first 32-k block (substeps 0, 1), s16 =
  // d of the second, zs / zh = 128 d (d rounded to bf16 first); kQ4_0 (lane
  // kq: block kq): sc = d, s16 = d / 16, zs = zh = 8 d
  auto convert_scales = [&](int set, int gq) {
    if constexpr (WF == kQ8_0 || WF == kQ4_0) {
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const uint4 h = hq_raw[j];
        const uint32_t w = gq == 0 ? h.x : gq == 1 ? h.y : gq == 2 ? h.z : h.w;
        if constexpr (WF == kQ8_0) {
          const float d0 = ub_bf16_to_f32(ub_f32_to_bf16(ub_f16_to_f32((uint16_t)(w & 0xffff))));
          const float d1 = ub_bf16_to_f32(ub_f32_to_bf16(ub_f16_to_f32((uint16_t)(w >> 16))));
          sc[set][j] = d0;
          zs[set][j] = 128.0f * d0;
          s16[set][j] = d1;
          zh[set][j] = 128.0f * d1;
        } else {
          const float d = ub_f16_to_f32((uint16_t)(kq ? w >> 16 : w & 0xffff));
          sc[set][j] = d;
          s16[set][j] = d * 0.0625f;
          zs[set][j] = 8.0f * d;
          zh[set][j] = 8.0f * d;
        }
      }
      return;
    }
    if constexpr (WF == kQ4K) {
      // gq is wave-uniform: one scalar branch, constant byte positions
#pragma unroll
      for (int j = 0; j < TN; j++) {
        float& a = sc[set][j];
        float& b = zs[set][j];
        float& c = s16[set][j];
        float& d = zh[set][j];
        switch (gq) {
          case 0: q4k_group<0>(hq_raw[j], a, b, c, d); break;
          case 1: q4k_group<1>(hq_raw[j], a, b, c, d); break;
          case 2: q4k_group<2>(hq_raw[j], a, b, c, d); break;
          default: q4k_group<3>(hq_raw[j], a, b, c, d); break;
        }
      }
      return;
    }
    const uint32_t sb[4] = {s_raw.x & 0xffff, s_raw.x >> 16, s_raw.y & 0xffff, s_raw.y >> 16};
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const float s = tof<DT>(sb[j]);
      sc[set][j] = s;
      if constexpr (WF == kGptq) {
        const uint32_t zw = z_raw >> (4 * (ncl & 7));
        s16[set][j] = s * 0.0625f;
        zs[set][j] = (float)((zw >> (4 * j)) & 15) * s;
      } else if constexpr (WF == kU4) {
        // z s is exact in f32 (8 + 8 or 11 + 11 significant bits), so
        // fma(q, s, -z s) rounds (q - z) s once, as the f32 subtract-then-
        // multiply of the reference does (q - z is exact)
        const uint32_t zb[4] = {zt_raw.x & 0xffff, zt_raw.x >> 16, zt_raw.y & 0xffff,
                                zt_raw.y >> 16};
        zs[set][j] = tof<DT>(zb[j]) * s;
        s16[set][j] = s * 0.0625f;
      } else {
        zs[set][j] = 128.0f * s;
      }
    }
  };
  uint32_t m_lo = 0x0f0f0f0fu, m_hi = 0xf0f0f0f0u, m_sg = 0x80808080u;
  asm volatile("" : "+v"(m_lo), "+v"(m_hi), "+v"(m_sg));
  // Raw words -> the lane's B operands (8 k of one column each, pairs of T).
  // The empty asm pins the results where they are computed: without it the
  // converts would be sunk next to the MFMAs that consume them, a substep
  // later, where nothing hides them.
  auto dequant = [&](int buf, int set, bool upper) {
    if constexpr (kNib32(WF)) {
      // substeps 0, 1: low nibbles, y = d sc q - dmin m; 2, 3: high nibbles
      // taken as 16 q and scaled by d sc / 16 (exact); one rounding to bf16
#pragma unroll
      for (int j = 0; j < TN; j++) {
        uint32_t o[4];
#pragma unroll
        for (int w = 0; w < 2; w++) {
          const u8x4 Q = __builtin_bit_cast(u8x4, bw[buf][2 * j + w] & (upper ? m_hi : m_lo));
          const float f = upper ? s16[set][j] : sc[set][j], z = upper ? zh[set][j] : zs[set][j];
          o[2 * w] = pack2<DT>(__builtin_fmaf((float)Q[0], f, -z), __builtin_fmaf((float)Q[1], f, -z));
          o[2 * w + 1] = pack2<DT>(__builtin_fmaf((float)Q[2], f, -z), __builtin_fmaf((float)Q[3], f, -z));
        }
        bf[buf][j] = make_uint4(o[0], o[1], o[2], o[3]);
      }
    } else if constexpr (WF == kGptq) {
#pragma unroll
      for (int j = 0; j < TN; j++)
        bf[buf][j] = dequant_word<DT>(bw[buf][j], m_lo, m_hi, sc[set][j], s16[set][j], zs[set][j]);
    } else if constexpr (WF == kU4) {
      // word p = byte-row p of the unit (k 2p low nibble, 2p + 1 high), byte
      // c = column c: T((q - z) s) as one fma from the exact z s (the high
      // nibble enters as 16 q against s / 16)
      u8x4 L[4], H[4];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t w = TN == 4 ? bw[buf][q] : bw[buf][q] >> bsh;
        L[q] = __builtin_bit_cast(u8x4, w & m_lo);
        H[q] = __builtin_bit_cast(u8x4, w & m_hi);
      }
#pragma unroll
      for (int j = 0; j < TN; j++) {
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float lo = __builtin_fmaf((float)L[q][j], sc[set][j], -zs[set][j]);
          const float hi = __builtin_fmaf((float)H[q][j], s16[set][j], -zs[set][j]);
          o[q] = pack2<DT>(lo, hi);
        }
        bf[buf][j] = make_uint4(o[0], o[1], o[2], o[3]);
      }
    } else {
      // int8 as q + 128 (sign bit flipped): fma(q + 128, s, -128 s) = q s
      // exactly, one rounding to T (kQ8_0: the block's d by substep)
      constexpr int NWD = 8;
      u8x4 X[NWD];
      if constexpr (WF == kI8Kn) {
#pragma unroll
        for (int q = 0; q < NWD; q++)
          X[q] = __builtin_bit_cast(u8x4, (TN == 4 ? bw[buf][q] : bw[buf][q] >> bsh) ^ m_sg);
      } else {
#pragma unroll
        for (int q = 0; q < 2 * TN; q++) X[q] = __builtin_bit_cast(u8x4, bw[buf][q] ^ m_sg);
      }
#pragma unroll
      for (int j = 0; j < TN; j++) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
          // kI8Kn: k row e of column j; kI8Nk: byte e of column j's 8
          const float x = WF == kI8Kn ? (float)X[e][j] : (float)X[2 * j + (e >> 2)][e & 3];
          if constexpr (WF == kQ8_0)
            v[e] = __builtin_fmaf(x, upper ? s16[set][j] : sc[set][j], upper ? -zh[set][j] : -zs[set][j]);
          else
            v[e] = __builtin_fmaf(x, sc[set][j], -zs[set][j]);
        }
        bf[buf][j] = make_uint4(pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]),
                                pack2<DT>(v[4], v[5]), pack2<DT>(v[6], v[7]));
      }
    }
#pragma unroll
    for (int j = 0; j < TN; j++)
      asm volatile("" : "+v"(bf[buf][j].x), "+v"(bf[buf][j].y), "+v"(bf[buf][j].z), "+v"(bf[buf][j].w));
  };
  auto mfmas = [&](int abuf, int bbuf) {
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++) acc[i][j] = mfma<DT>(af[abuf][i], bf[bbuf][j], acc[i][j]);
  };
  // The weight words go out before the A fragments in every substep: the
  // next substep's dequant waits for them, and the in-order LDS counter then
  // lets the A reads stay in flight.
  // Issue is in order per wave.  Each substep is its own scheduling region:
  // its MFMAs alternate with its LDS reads (for two substeps ahead; one after
  // each of MFMAs 1..6) and the next substep's dequant VALU, which executes
  // while the matrix pipe is busy.  (Measured: reads spread this way beat
  // issuing them all first by ~4%.)
  constexpr int NBR = WF == kGptq || WF == kU4 ? 1 : WF == kI8Kn ? 2 : TN;  // B reads
  constexpr int VPM = WF == kGptq || kNib32(WF) ? 8 : 12;  // VALU per MFMA slot
  auto sched = [&]() {
#pragma unroll
    for (int q = 0; q < TM * TN; q++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
      if (q >= 1 && q < 2 + NBR + TM) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
      __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);  // VALU
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // ---- prologue: stages 0..NSTG-1 in flight; wait for stage 0
  issue(0, sbase);
  if (nkh > 1) issue(1, sbase + STB);
  if (NSTG == 3 && nkh > 2) issue(2, sbase + 2 * STB);
  if (NSTG == 3 && nkh > 2) ub_wait_vmcnt<2 * NL>();
  else if (nkh > 1) ub_wait_vmcnt<NL>();
  else ub_wait_vmcnt<0>();
  ub_barrier();
  read_scales(sbase, 0);
  convert_scales(0, (kb + kh * nkh) & 3);
  read_b(sbase, 0, 0);
  read_a(sbase, 0, 0);
  read_b(sbase, 1, 1);
  read_a(sbase, 1, 1);
  dequant(0, 0, false);

  // ---- K-step t from stage `cur`; stage `nxt` holds t + 1 (stale at the
  // last step: those prefetches go unused).  Substep s: MFMAs on af[s] and
  // bf[s & 1]; reads of substep s + 2 into af[(s + 2) & 3] / bw[s & 1];
  // dequant of substep s + 1.
  auto kstep = [&](int t, uint32_t cur, uint32_t nxt) {
    read_b(cur, 2, 0);
    read_a(cur, 2, 2);
    mfmas(0, 0);
    dequant(1, 0, false);
    sched();

    read_b(cur, 3, 1);
    read_a(cur, 3, 3);
    mfmas(1, 1);
    dequant(0, 0, true);
    sched();

    // every wave is past its last read of `cur`; stage t + 1 has landed
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    if (NSTG == 3 && t + 2 < nkh) ub_wait_vmcnt<NL>();
    else ub_wait_vmcnt<0>();
    ub_barrier();
    if (t + NSTG < nkh) issue(t + NSTG, cur);

    read_b(nxt, 0, 0);
    read_scales(nxt, t + 1);
    read_a(nxt, 0, 0);
    mfmas(2, 0);
    dequant(1, 0, true);
    sched();

    read_b(nxt, 1, 1);
    read_a(nxt, 1, 1);
    mfmas(3, 1);
    convert_scales(1, (t + 1 + kb + kh * nkh) & 3);
    dequant(0, 1, false);
    sched();
#pragma unroll
    for (int j = 0; j < TN; j++) {
      sc[0][j] = sc[1][j];
      s16[0][j] = s16[1][j];
      zs[0][j] = zs[1][j];
      zh[0][j] = zh[1][j];
    }
  };
  for (int t = 0; t < nkh; t++) {
    const int c = t % NSTG;
    kstep(t, sbase + c * STB, sbase + (c == NSTG - 1 ? 0 : c + 1) * STB);
  }

  // ---- split-K: the upper-K wavefronts hand their sums to the lower-K ones
  if constexpr (KS == 2) {
    __syncthreads();
    float4* red = (float4*)smem;
    if (kh == 1) {
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const f32x16& v = acc[i][j];
            red[(((i * TN + j) * 4 + r) * NWN + wn) * 64 + lane] =
                make_float4(v[4 * r], v[4 * r + 1], v[4 * r + 2], v[4 * r + 3]);
          }
    }
    __syncthreads();
    if (kh == 1) return;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float4 v = red[(((i * TN + j) * 4 + r) * NWN + wn) * 64 + lane];
          acc[i][j][4 * r] += v.x;
          acc[i][j][4 * r + 1] += v.y;
          acc[i][j][4 * r + 2] += v.z;
          acc[i][j][4 * r + 3] += v.w;
        }
  }

  // ---- epilogue: lane l, register r of tile (i, j) holds
  // C[wm*128 + 32 i + 8 (r / 4) + 4 (l / 32) + r % 4][n0 + ncl + j]
  uint16_t* C = (uint16_t*)p.c;
  const int n = n0 + ncl;
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int m = m0 + wm * WR + 32 * i + 8 * (r >> 2) + 4 * kq + (r & 3);
      if (m < M && n < N) {  // N % 8 == 0: all TN columns are in range
        if (S > 1) {
          float* P = p.part + ((size_t)blockIdx.y * M + m) * N + n;
          if constexpr (TN == 4)
            *(float4*)P = make_float4(acc[i][0][r], acc[i][1][r], acc[i][2][r], acc[i][3][r]);
          else
            *(float2*)P = make_float2(acc[i][0][r], acc[i][1][r]);
        } else if (kGguf(WF) && p.c_f32) {
          float* Cf = (float*)p.c + (size_t)m * N + n;
          if constexpr (TN == 4)
            *(float4*)Cf = make_float4(acc[i][0][r], acc[i][1][r], acc[i][2][r], acc[i][3][r]);
          else
            *(float2*)Cf = make_float2(acc[i][0][r], acc[i][1][r]);
        } else if constexpr (TN == 4)
          *(uint2*)(C + (size_t)m * N + n) = make_uint2(pack2<DT>(acc[i][0][r], acc[i][1][r]),
                                                        pack2<DT>(acc[i][2][r], acc[i][3][r]));
        else
          *(uint32_t*)(C + (size_t)m * N + n) = pack2<DT>(acc[i][0][r], acc[i][1][r]);
      }
    }
}

// 64-row tiles (TMX = 2) for the split variant up to 64 rows (two of them
// for 65..128 rows measured level with one 128-row tile: 4096 x 14336 GPTQ,
// 80 tokens 29.7 against 27.0 us, 128 tokens 31.1 against 32.9)
bool small_tiles(int M) { return M <= 64; }

template <int WF, int DT, int WM, int KS, int NSTG>
int launch(const W4Args& a, hipStream_t s) {
  const int path = WF == kGptq ? ub_tune(UB_TUNE_W4A16_PATH) : 0;
  if constexpr (WF == kGptq && NSTG == 3) {
    if (path == 5 && WM == 2) {  // 256 x 256 as four 256 x 64 wave tiles
      dim3 grid(ub_cdiv(a.N, kBN) * ub_cdiv(a.M, 256), a.ksplit > 1 ? a.ksplit : 1);
      k_w4a16<WF, DT, 1, 1, 4, 8><<<grid, 256, 0, s>>>(a);
      return ub_check_launch("w4a16 gemm");
    }
    if (path == 3) {
      dim3 grid(ub_cdiv(a.N, kBN) * ub_cdiv(a.M, 128 * WM), a.ksplit > 1 ? a.ksplit : 1);
      k_w4a16<WF, DT, WM, KS, 4><<<grid, 256, 0, s>>>(a);
      return ub_check_launch("w4a16 gemm");
    }
  }
  if constexpr (WM == 1 && KS == 2) {
    if (small_tiles(a.M)) {  // 64-row tiles: at most 64 padding rows per tile
      dim3 grid(ub_cdiv(a.N, kBN) * ub_cdiv(a.M, 64), a.ksplit > 1 ? a.ksplit : 1);
      k_w4a16<WF, DT, 1, 2, 8, 2, NSTG><<<grid, 512, 0, s>>>(a);
      return ub_check_launch("w4a16 gemm");
    }
  }
  dim3 grid(ub_cdiv(a.N, kBN) * ub_cdiv(a.M, 128 * WM), a.ksplit > 1 ? a.ksplit : 1);
  k_w4a16<WF, DT, WM, KS, 8, 4, NSTG><<<grid, 512, 0, s>>>(a);
  return ub_check_launch("w4a16 gemm");
}

int num_cus() {
  static int n = 0;
  if (n == 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      n = v;
    else
      n = 256;
  }
  return n;
}

// Tile 256 x 256 (2 x 2 wavefronts) or 128 x 256 with K split over two
// wavefront pairs: whichever keeps more of the CUs busy over the launch's
// rounds (ties: the taller tile, which reads half the weight per flop).
// force: 0 shape rule, 1 split, 2 no split.
bool pick_split(int M, int N, int K, int force) {
  const bool can_split = K % 128 == 0;
  if (force == 1) return can_split;
  if (force == 2 || !can_split) return false;
  const long cus = num_cus(), tn = ub_cdiv(N, kBN);
  const long t256 = ub_cdiv(M, 256) * tn, t128 = ub_cdiv(M, 128) * tn;
  const double f256 = (double)M / (256.0 * ub_cdiv(M, 256)) * t256 / (double)(ub_cdiv(t256, cus) * cus);
  const double f128 = (double)M / (128.0 * ub_cdiv(M, 128)) * t128 / (double)(ub_cdiv(t128, cus) * cus);
  return f128 > f256 + 1e-9;
}

template <int WF>
int dispatch_wf(const W4Args& p, int dtype, bool split, hipStream_t s) {
  // int8 weights: a split stage holds 66 KB (Q4_K 56 KB), so that variant keeps 2 stages
  constexpr int NS2 = WF == kI8Kn || WF == kI8Nk || kGguf(WF) ? 2 : 3;
  if constexpr (kGguf(WF)) {
    return split ? launch<WF, UB_BF16, 1, 2, NS2>(p, s) : launch<WF, UB_BF16, 2, 1, 3>(p, s);
  } else {
    if (dtype == UB_BF16)
      return split ? launch<WF, UB_BF16, 1, 2, NS2>(p, s) : launch<WF, UB_BF16, 2, 1, 3>(p, s);
    return split ? launch<WF, UB_F16, 1, 2, NS2>(p, s) : launch<WF, UB_F16, 2, 1, 3>(p, s);
  }
}

int gemm_tile_force() {
  const int t = ub_tune(UB_TUNE_GEMM_TILE);
  return t == 1 ? 1 : t == 3 ? 2 : 0;
}

// out[i] = sum over s = 0..S-1 of part[s][i], in that order (f32), as f32
// (DT = UB_F32) or rounded once to T; 4 elements per thread, the S loads
// unrolled so that they are all in flight together.
template <int DT, int S>
__global__ void __launch_bounds__(256) k_ksum(const float* __restrict__ part, size_t n4,
                                              void* __restrict__ out) {
  const size_t i = blockIdx.x * (size_t)256 + threadIdx.x;
  if (i >= n4) return;
  float4 v[S];
#pragma unroll
  for (int s = 0; s < S; s++) v[s] = ((const float4*)part)[(size_t)s * n4 + i];
  float4 a = v[0];
#pragma unroll
  for (int s = 1; s < S; s++) a.x += v[s].x, a.y += v[s].y, a.z += v[s].z, a.w += v[s].w;
  if constexpr (DT == UB_F32) {
    ((float4*)out)[i] = a;
  } else {
    const uint32_t lo = (uint32_t)(DT == UB_F16 ? ub_f32_to_f16(a.x) : ub_f32_to_bf16(a.x)) |
                        ((uint32_t)(DT == UB_F16 ? ub_f32_to_f16(a.y) : ub_f32_to_bf16(a.y)) << 16);
    const uint32_t hi = (uint32_t)(DT == UB_F16 ? ub_f32_to_f16(a.z) : ub_f32_to_bf16(a.z)) |
                        ((uint32_t)(DT == UB_F16 ? ub_f32_to_f16(a.w) : ub_f32_to_bf16(a.w)) << 16);
    ((uint2*)out)[i] = make_uint2(lo, hi);
  }
}

// Split over K across workgroups for grids that leave CUs idle: with fewer
// tiles than half the CUs, each tile's K range is cut in S = 2, 4 or 8 parts
// (tiles x S <= CUs), the parts' f32 sums go to the stream's workspace and
// k_ksum adds them in a fixed order.  S = 1 where K does not divide (the
// GGUF formats: whole 256-k spans per part) or the call may not allocate
// (may_alloc false: the allocation-free entry point).
// MI355X, 4096 x 14336 GPTQ at 64 / 256 tokens: 56 / 112 tiles.
int pick_ksplit(const W4Args& p, bool split, bool gguf, bool may_alloc) {
  if (!may_alloc || ub_tune(UB_TUNE_W4A16_PATH) == 7) return 1;
  const int KS = split ? 2 : 1;
  const long tiles = (long)ub_cdiv(p.M, split ? (small_tiles(p.M) ? 64 : 128) : 256) * ub_cdiv(p.N, kBN);
  const long cus = num_cus();
  int S = 1;
  while (S < 8 && tiles * S * 2 <= cus && (p.K / 64) % (S * 2 * KS) == 0 &&
         (!gguf || (p.K / 256) % (S * 2) == 0))
    S *= 2;
  return S;
}

// Scratch for the K split picked above (none when S == 1); sets p.ksplit and
// p.part, or leaves the launch unsplit when the allocation fails.
struct KSplit {
  UbScratch ws;
  KSplit(W4Args& p, int S, hipStream_t s) : ws(s, S > 1 ? (size_t)S * p.M * p.N * 4 : 0) {
    p.ksplit = S > 1 && ws.get() ? S : 1;
    p.part = p.ksplit > 1 ? (float*)ws.get() : nullptr;
  }
};

int ksum_launch(const W4Args& p, int out_dt, hipStream_t s) {
  if (p.ksplit <= 1) return UB_OK;
  const size_t n4 = (size_t)p.M * p.N / 4;
  const unsigned g = (unsigned)((n4 + 255) / 256);
#define UB_KS(DT)                                                                  \
  if (p.ksplit == 2) k_ksum<DT, 2><<<g, 256, 0, s>>>(p.part, n4, p.c);             \
  else if (p.ksplit == 4) k_ksum<DT, 4><<<g, 256, 0, s>>>(p.part, n4, p.c);        \
  else k_ksum<DT, 8><<<g, 256, 0, s>>>(p.part, n4, p.c);
  if (out_dt == UB_F32) { UB_KS(UB_F32) }
  else if (out_dt == UB_F16) { UB_KS(UB_F16) }
  else { UB_KS(UB_BF16) }
#undef UB_KS
  return ub_check_launch("w4a16 k-split sum");
}

}  // namespace

// Pipelined W4A16 GEMM; returns UB_ERR_UNSUPPORTED (without recording an
// error) when the shape is outside its contract or a is not 16-byte aligned
// (its rows reach LDS by 16-byte direct-to-LDS loads), so the caller can
// fall back.
int ub_w4a16_pipelined(const void* a, const int32_t* qw, const void* scales, const int32_t* qzeros,
                       void* out, int M, int K, int N, int group, int dtype, hipStream_t s) {
  if (group % 64 != 0 || K % 64 != 0 || K < 64 || N % 8 != 0 || ((uintptr_t)a & 15) != 0)
    return UB_ERR_UNSUPPORTED;
  if ((uint64_t)M * K * 2 >= 0x80000000ull || (uint64_t)(K / 8) * N * 4 >= 0x80000000ull ||
      (uint64_t)(K / group) * N * 2 >= 0x80000000ull)
    return UB_ERR_UNSUPPORTED;  // 32-bit buffer offsets
  W4Args p{a, qw, scales, qzeros, out, M, N, K, group};
  const bool split = pick_split(M, N, K, gemm_tile_force());
  KSplit ks(p, pick_ksplit(p, split, false, true), s);
  const int e = dispatch_wf<kGptq>(p, dtype, split, s);
  return e ? e : ksum_launch(p, dtype, s);
}

// 1 when the shape rule picks the 128 x 256 split-K tile (for the GEMM
// launch-parameter getter).
int ub_wq_split(int M, int N, int K) { return pick_split(M, N, K, gemm_tile_force()) ? 1 : 0; }

// The same pipeline for the reference-layout weights of matmul_*_{4,8}bit
// (wf = 1: uint8 [K/2, N] with T zeros; 2: int8 [K, N]; 3: int8 [N, K]).
// tile: 0 shape rule, 1 the 128 x 256 split-K tile, 2 the 256 x 256 tile.
int ub_wq_pipelined(int wf, const void* a, const void* w, const void* scales, const void* zeros,
                    void* out, int M, int K, int N, int group, int dtype, int tile, hipStream_t s) {
  if (group % 64 != 0 || K % 64 != 0 || K < 64 || N % 8 != 0 || wf < 1 || wf > 3 ||
      ((uintptr_t)a & 15) != 0)
    return UB_ERR_UNSUPPORTED;
  if ((uint64_t)M * K * 2 >= 0x80000000ull || (uint64_t)K * N >= 0x80000000ull ||
      (uint64_t)(K / group) * N * 2 >= 0x80000000ull)
    return UB_ERR_UNSUPPORTED;  // 32-bit buffer offsets
  W4Args p{a, w, scales, zeros, out, M, N, K, group};
  const bool split = pick_split(M, N, K, tile ? tile : gemm_tile_force());
  KSplit ks(p, pick_ksplit(p, split, false, true), s);
  const int e = wf == kU4    ? dispatch_wf<kU4>(p, dtype, split, s)
                : wf == kI8Kn ? dispatch_wf<kI8Kn>(p, dtype, split, s)
                              : dispatch_wf<kI8Nk>(p, dtype, split, s);
  return e ? e : ksum_launch(p, dtype, s);
}

// GGUF weight [N, K] (qtype 2 Q4_0, 8 Q8_0, 12 Q4_K; SoA: the block headers,
// then the payloads) times bf16 x [M, K] -> y [M, N] (f32 when y_f32, else
// bf16): the same pipeline, the weight dequantized to the values of
// dequantize_block_*_bf16 in registers.  UB_ERR_UNSUPPORTED (nothing
// recorded) outside K % 256 == 0, N % 8 == 0 and 32-bit buffer offsets
// (ub_gguf_pipelined_fits), or for an x that is not 16-byte aligned (its
// rows reach LDS by 16-byte direct-to-LDS loads).
bool ub_gguf_pipelined_fits(int qtype, int M, int N, int K) {
  if (M < 1 || N < 8 || K < 256 || K % 256 != 0 || N % 8 != 0) return false;
  if (qtype != UB_Q4_K && qtype != UB_Q8_0 && qtype != UB_Q4_0) return false;
  const uint64_t hdr_b = (uint64_t)N * (K / 256) * 16;  // header bytes (all three)
  const uint64_t body_b = qtype == UB_Q8_0 ? (uint64_t)N * K : (uint64_t)N * K / 2;
  return (uint64_t)M * K * 2 < 0x80000000ull && hdr_b + body_b < 0x80000000ull;
}

int ub_gguf_pipelined(int qtype, const void* w, const void* x, void* y, int y_f32, int M, int N,
                      int K, bool may_alloc, hipStream_t s) {
  if (!ub_gguf_pipelined_fits(qtype, M, N, K) || ((uintptr_t)x & 15) != 0)
    return UB_ERR_UNSUPPORTED;
  const uint64_t hdr_b = (uint64_t)N * (K / 256) * 16;
  const uint8_t* hdr = (const uint8_t*)w;
  W4Args p{x, hdr + hdr_b, nullptr, hdr, y, M, N, K, 256, y_f32};
  const bool split = pick_split(M, N, K, gemm_tile_force());
  KSplit ks(p, pick_ksplit(p, split, true, may_alloc), s);
  const int e = qtype == UB_Q4_K   ? dispatch_wf<kQ4K>(p, UB_BF16, split, s)
                : qtype == UB_Q8_0 ? dispatch_wf<kQ8_0>(p, UB_BF16, split, s)
                                   : dispatch_wf<kQ4_0>(p, UB_BF16, split, s);
  return e ? e : ksum_launch(p, y_f32 ? UB_F32 : UB_BF16, s);
}
