// moe.hip -- MoE routing and grouped expert GEMM for gfx950.
//
//   topk_softmax_{f32,f16,bf16}   topk_softmax_host.cpp:103-208
//   moe_align_block_size          moe_align_host.cpp:51-935
//   invoke_fused_moe_{bf16,f16}   fused_moe_host.cpp:43-536  (+ W8A16 variant)
//   silu_and_mul / moe_sum        the steps either side of the grouped GEMM
//   moe_{f16,bf16}, indexed_moe_{f16,bf16}   moe_host.cpp:27-293 (legacy)
//
// Device-side argument errors (expert ids out of range, bad real_token_num)
// do not trap as the reference's op_assert does: the kernel leaves a "no
// work" result (num_tokens_post_pad = 0) and raises a device flag that
// ubridge_device_error() reads after synchronizing the stream.
#include "common.h"
#include "lds_dma.h"
#include "registry.h"

#include <algorithm>

namespace {

__device__ int g_device_error;  // UB_ERR_* set by kernels, read by ubridge_device_error

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kOOB = 0x80000000u;

template <int DT>
__device__ __forceinline__ float tof(uint16_t b) {
  if constexpr (DT == UB_BF16) return ub_bf16_to_f32(b);
  else return ub_f16_to_f32(b);
}
template <int DT>
__device__ __forceinline__ uint16_t fromf(float v) {
  if constexpr (DT == UB_BF16) return __builtin_bit_cast(unsigned short, (__bf16)v);
  else return __builtin_bit_cast(unsigned short, (_Float16)v);
}

// =============================================================== top-k softmax
// Reference order: max, sum of expf(v - max), p = expf(v - max) * (1/sum);
// k rounds of arg-max over p (largest value, lowest index on ties); outputs
// rounded to T; with norm, each T-rounded weight is scaled by 1/(sum of the
// f32 picks) and rounded again.
// A token is handled by a group of G lanes (G = 16: four tokens per
// wavefront, for E <= 256 and k <= 16; else G = 64), each lane keeping its
// NPL probabilities (experts lane + G j) in registers.  A round is two group
// reductions by DPP row ops (and permlane swaps for G = 64): the max of the
// lanes' best values, then the min expert index among the lanes holding it.
// The next token's logits are loaded while the current one is reduced.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
template <int G, int OP>  // OP 0: f32 max, 1: u32 min, 2: f32 sum
__device__ __forceinline__ uint32_t group_reduce(uint32_t v) {
  auto op = [](uint32_t a, uint32_t b) -> uint32_t {
    if constexpr (OP == 0) return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
    else if constexpr (OP == 1) return a < b ? a : b;
    else return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
  };
  v = op(v, dpp_u<0xB1>(v));   // quad_perm [1,0,3,2]
  v = op(v, dpp_u<0x4E>(v));   // quad_perm [2,3,0,1]
  v = op(v, dpp_u<0x141>(v));  // row_half_mirror
  v = op(v, dpp_u<0x140>(v));  // row_mirror
  if constexpr (G == 64) {
    auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = op(r[0], r[1]);
    auto r2 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    v = op(r2[0], r2[1]);
  }
  return v;
}

template <int DT, int G, int NPL>
__device__ __forceinline__ void topk_load(const void* __restrict__ in, int t, int T, int E, int gl,
                                          float (&v)[NPL]) {
  const size_t base = (size_t)(t < T ? t : 0) * E;
#pragma unroll
  for (int j = 0; j < NPL; j++) {
    const int e = gl + G * j;
    float x = -INFINITY;
    if (t < T && e < E) {
      if constexpr (DT == UB_F32) x = ((const float*)in)[base + e];
      else x = tof<DT>(((const uint16_t*)in)[base + e]);
    }
    v[j] = x;
  }
}

// Top-k of token t (logits v, loaded by topk_load) by the G lanes of a
// group; gl = lane index in the group.  Writes T weights and ids as the
// reference does; if wf32 is given, also the f32 value of every final T
// weight (the grouped GEMM's routed-weight operand); if tei is given, the
// source row j * T + t of slot (t, j) (the token_expert_indices output of
// the status-returning topk entry).  Pick jj is held by group lane jj until
// the end.
template <int DT, int G, int NPL>
__device__ __forceinline__ void topk_token(float (&p)[NPL], void* __restrict__ out,
                                           int* __restrict__ idx, float* __restrict__ wf32,
                                           int* __restrict__ tei, int t, int T, int E, int k,
                                           int norm, int gl) {
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < NPL; j++) mx = fmaxf(mx, p[j]);
  mx = __uint_as_float(group_reduce<G, 0>(__float_as_uint(mx)));
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < NPL; j++)
    if (gl + G * j < E) sum += expf(p[j] - mx);
  sum = __uint_as_float(group_reduce<G, 2>(__float_as_uint(sum)));
  const float inv = sum > 0.f ? 1.f / sum : 1.f;
#pragma unroll
  for (int j = 0; j < NPL; j++) p[j] = gl + G * j < E ? expf(p[j] - mx) * inv : -INFINITY;
  float wsum = 0.f, picked = 0.f;
  int got = 0, pidx = 0;
  for (int jj = 0; jj < k; jj++) {
    float best = -INFINITY;
    int bj = 0;
#pragma unroll
    for (int j = 0; j < NPL; j++)
      if (p[j] > best) { best = p[j]; bj = j; }  // first (lowest e) on ties within the lane
    const float wb = __uint_as_float(group_reduce<G, 0>(__float_as_uint(best)));
    if (wb == -INFINITY) break;  // fewer than k finite candidates
    const uint32_t cand = best == wb ? (uint32_t)(gl + G * bj) : 0xffffffffu;
    const int bi = (int)group_reduce<G, 1>(cand);
    if (gl == bi % G) {
#pragma unroll
      for (int j = 0; j < NPL; j++)
        if (j == bi / G) p[j] = -INFINITY;
    }
    if (gl == jj) { picked = wb; pidx = bi; }
    wsum += wb;
    got++;
  }
  if (gl < got) {
    const size_t o = (size_t)t * k + gl;
    float w = picked;
    uint16_t wt = 0;
    if constexpr (DT != UB_F32) { wt = fromf<DT>(w); w = tof<DT>(wt); }
    if (norm && wsum > 0.f) {
      w = w * (1.f / wsum);
      if constexpr (DT != UB_F32) { wt = fromf<DT>(w); w = tof<DT>(wt); }
    }
    if constexpr (DT == UB_F32) ((float*)out)[o] = w;
    else ((uint16_t*)out)[o] = wt;
    idx[o] = pidx;
    if (wf32) wf32[o] = w;
    if (tei) tei[o] = gl * T + t;
  }
}

// Every group of G lanes of the launch walks tokens g, g + ngroups, ...
template <int DT, int G, int NPL>
__device__ __forceinline__ void topk_tokens(const void* __restrict__ in, void* __restrict__ out,
                                            int* __restrict__ idx, float* __restrict__ wf32,
                                            int* tei, int g, int ngroups, int T, int E, int k,
                                            int norm, int gl) {
  float cur[NPL], nxt[NPL];
  topk_load<DT, G, NPL>(in, g, T, E, gl, cur);
  for (int t = g; t < T; t += ngroups) {
    topk_load<DT, G, NPL>(in, t + ngroups, T, E, gl, nxt);
    topk_token<DT, G, NPL>(cur, out, idx, wf32, tei, t, T, E, k, norm, gl);
#pragma unroll
    for (int j = 0; j < NPL; j++) cur[j] = nxt[j];
  }
}

template <int DT, int G, int NPL>
__global__ void __launch_bounds__(256) k_topk_softmax(const void* __restrict__ in,
                                                      void* __restrict__ out,
                                                      int* __restrict__ idx,
                                                      float* __restrict__ wf32,
                                                      int* __restrict__ tei, int T, int E, int k,
                                                      int norm) {
  const int gpb = 256 / G;  // groups per workgroup
  const int g = blockIdx.x * gpb + threadIdx.x / G;
  topk_tokens<DT, G, NPL>(in, out, idx, wf32, tei, g, gridDim.x * gpb, T, E, k, norm,
                          threadIdx.x % G);
}

template <int DT>
int topk_softmax_launch(const void* in, void* out, int* idx, int T, int E, int k, int norm,
                        void* stream, const char* nm, float* wf32 = nullptr,
                        int* tei = nullptr) {
  UB_REQUIRE(T >= 0 && E > 0 && E <= 4096 && k > 0 && k <= E && k <= 64,
             "%s: T=%d E=%d k=%d (E <= 4096, 0 < k <= min(E, 64))", nm, T, E, k);
  if (T == 0) return UB_OK;
  UB_REQUIRE(in && out && idx, "%s: null pointer", nm);
  hipStream_t s = ub_stream(stream);
  // groups walk the tokens with a stride of the grid's group count
#define UB_TOPK(G_, NPL_)                                                                 \
  {                                                                                       \
    const int gpb = 256 / G_;                                                             \
    const dim3 g((unsigned)std::min<long>(ub_cdiv(T, gpb), 1024));                        \
    k_topk_softmax<DT, G_, NPL_><<<g, 256, 0, s>>>(in, out, idx, wf32, tei, T, E, k, norm); \
  }
  // a wavefront per token up to 128 experts (measured on MI355X at 256
  // tokens x 128 experts, top-8: 3.9 us against 5.0 us for 16-lane groups
  // holding 8 logits each: the per-round arg-max over a lane's values is the
  // longer chain)
  if (E <= 64) UB_TOPK(64, 1)
  else if (E <= 128) UB_TOPK(64, 2)
  else if (k <= 16 && E <= 256) UB_TOPK(16, 16)
  else if (E <= 256) UB_TOPK(64, 4)
  else if (E <= 512) UB_TOPK(64, 8)
  else if (E <= 1024) UB_TOPK(64, 16)
  else UB_TOPK(64, 64)
#undef UB_TOPK
  return ub_check_launch(nm);
}

// ============================================================ moe_align_block_size
// One workgroup of 1024 threads (16 wavefronts) for any slot count.  The
// slots i = t*k + j are cut into chunks of 64 (one wavefront-wide load);
// wavefront w takes a contiguous run of chunks.  Within a chunk the lanes
// holding the same expert are found by one ballot per bit of the expert id,
// so a slot's rank among equal experts earlier in the chunk is a popcount.
// Pass 1 counts each wavefront's slots per expert (LDS row per wavefront,
// updated by the first lane of each expert group; no atomics); the counts
// are prefixed over wavefronts per expert and the padded expert offsets
// scanned; pass 2 walks the same chunks again and places slot i at
// eoff[e] + (slots of e in earlier wavefronts and chunks) + rank.  Slots of
// one expert therefore keep ascending order, as the reference's stable
// scatter (moe_align_host.cpp:766-921).
constexpr int kAlignThreads = 1024, kAlignWaves = kAlignThreads / 64;

// lanes of this wavefront holding the same (non-negative) expert e
__device__ __forceinline__ uint64_t same_expert(int e, int nbits) {
  uint64_t m = __ballot(e >= 0);
  for (int b = 0; b < nbits; b++) {
    const bool bit = (e >> b) & 1;
    const uint64_t on = __ballot(bit);
    m &= bit ? on : ~on;
  }
  return m;
}

__global__ void __launch_bounds__(kAlignThreads) k_moe_align(
    int* __restrict__ sorted, int* __restrict__ experts, int* __restrict__ ntpp,
    const int* __restrict__ ids, const int* __restrict__ real_tn, const int* __restrict__ emap,
    int E, int bs, int T, int k) {
  extern __shared__ int sh[];
  int* wcnt = sh;                    // [kAlignWaves][E]
  int* eoff = wcnt + kAlignWaves * E;  // [E + 1]
  __shared__ int bad;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int pad = T * k;
  const int max_padded = T * k + E * (bs - 1);
  const int max_blocks = max_padded / bs;
  const int nbits = E > 1 ? 32 - __clz(E - 1) : 0;
  if (tid == 0) bad = 0;
  for (int i = tid; i < kAlignWaves * E; i += kAlignThreads) wcnt[i] = 0;
  __syncthreads();
  int tn = T;
  if (real_tn) {
    tn = *real_tn;
    if (tn < 0 || tn > T) { if (tid == 0) bad = 1; tn = 0; }
  }
  const int n = tn * k;
  if (emap)
    for (int e = tid; e < E; e += kAlignThreads)
      if (emap[e] < -1 || emap[e] >= E) bad = 1;
  // pad fill of both outputs (memsets at moe_align_host.cpp:777-784)
  for (int i = tid; i < max_padded; i += kAlignThreads) sorted[i] = pad;
  for (int i = tid; i < max_blocks; i += kAlignThreads) experts[i] = 0;
  const int nc = (n + 63) / 64, cpw = (nc + kAlignWaves - 1) / kAlignWaves;
  const int c0 = wv * cpw, c1 = min(nc, c0 + cpw);
  int* mine = wcnt + wv * E;
  const uint64_t below = (1ull << lane) - 1;
  // the wavefront's ids, KB chunks at a time (independent loads in flight)
  constexpr int KB = 8;
  auto load_ids = [&](int cb, int (&ev)[KB]) {
#pragma unroll
    for (int q = 0; q < KB; q++) {
      const int i = (cb + q) * 64 + lane;
      ev[q] = cb + q < c1 && i < n ? ids[i] : -1;
    }
  };
  // pass 1: this wavefront's count per expert (and the id check)
  bool any_bad = false;
  for (int cb = c0; cb < c1; cb += KB) {
    int ev[KB];
    load_ids(cb, ev);
#pragma unroll
    for (int q = 0; q < KB; q++) {
      if (cb + q >= c1) break;
      const int i = (cb + q) * 64 + lane;
      any_bad |= i < n && (ev[q] < 0 || ev[q] >= E);
      const int e = ev[q] >= 0 && ev[q] < E ? ev[q] : -1;
      const uint64_t m = same_expert(e, nbits);
      if (e >= 0 && __popcll(m & below) == 0) mine[e] += __popcll(m);
    }
  }
  if (any_bad) bad = 1;
  __syncthreads();
  if (bad) {
    if (tid == 0) {
      ntpp[0] = 0;
      g_device_error = UB_ERR_INDEX;
    }
    return;
  }
  // exclusive prefix over wavefronts per expert; padded totals
  for (int e = tid; e < E; e += kAlignThreads) {
    int run = 0;
    for (int w = 0; w < kAlignWaves; w++) {
      const int v = wcnt[w * E + e];
      wcnt[w * E + e] = run;
      run += v;
    }
    eoff[e + 1] = (run + bs - 1) / bs * bs;
  }
  __syncthreads();
  if (tid < 64) {  // inclusive scan of the padded counts, 64 at a time
    int carry = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + tid;
      int v = e < E ? eoff[e + 1] : 0;
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(v, o, 64);
        if (tid >= o) v += u;
      }
      if (e < E) eoff[e + 1] = carry + v;
      carry += __shfl(v, 63, 64);
    }
    if (tid == 0) eoff[0] = 0;
  }
  __syncthreads();
  const int total = eoff[E];
  // pass 2: place every slot; the group's first lane advances the running count
  for (int cb = c0; cb < c1; cb += KB) {
    int ev[KB];
    load_ids(cb, ev);
#pragma unroll
    for (int q = 0; q < KB; q++) {
      if (cb + q >= c1) break;
      const int e = ev[q];
      const uint64_t m = same_expert(e, nbits);
      const int rank = __popcll(m & below);
      if (e >= 0) sorted[eoff[e] + mine[e] + rank] = (cb + q) * 64 + lane;
      __builtin_amdgcn_wave_barrier();  // every lane has read mine[e] before it moves
      if (e >= 0 && rank == 0) mine[e] += __popcll(m);
      __builtin_amdgcn_wave_barrier();
    }
  }
  // expert of every padded block: the e with eoff[e] <= b*bs < eoff[e+1]
  for (int b = tid; b < total / bs; b += kAlignThreads) {
    int lo = 0, hi = E;  // find last e with eoff[e] <= b*bs
    const int v = b * bs;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (eoff[mid] <= v) lo = mid; else hi = mid;
    }
    experts[b] = emap ? emap[lo] : lo;
  }
  if (tid == 0) ntpp[0] = total;
}

// ======================================== moe_align for small slot counts
// The same outputs as k_moe_align (no expert_map / real_token_num), for
// n = T*k <= 4096 slots in one workgroup of 1024 threads.  Slots are cut
// into chunks of 64, one wavefront-wide chunk per (wave, q).  Within a chunk
// the lanes holding the same expert are found by one ballot per bit of the
// expert id (log2 E ballots), so a slot's rank among equal experts before it
// is a popcount and the chunk's count per expert is written by the group's
// first lane.  The counts are prefixed over chunks per expert (in parallel
// chunk groups), the padded expert offsets come from one scan, and a slot's
// position is eoff[e] + (slots of e in earlier chunks) + rank: ascending
// slot order within each expert, as the reference.  No loop over the slots
// is serial.
constexpr int kRouteThreads = 1024, kRouteWaves = kRouteThreads / 64, kRouteMaxN = 4096;
constexpr int kRouteQ = kRouteMaxN / 64 / kRouteWaves;  // chunks per wave

// The align, by the whole 1024-thread workgroup; ids in global memory or
// LDS, sh the LDS scratch sized by align_small_lds.
__device__ __forceinline__ void align_small_body(const int* ids, int* sh, int* sorted, int* experts,
                                                 int* ntpp, int n, int E, int bs) {
  const int nc = (n + 63) / 64;
  // chunk groups for the prefix over chunks: G groups of CPG chunks per expert
  const int G = max(1, min(nc, kRouteThreads / E)), CPG = (nc + G - 1) / G;
  int* cnt = sh;             // [nc][E]: counts, then exclusive prefix over chunks
  int* part = cnt + nc * E;  // [G][E]: per-group sums, then their exclusive prefix
  int* eoff = part + G * E;  // [E + 1] padded expert offsets
  int& bad = eoff[E + 1];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int pad = n, max_padded = n + E * (bs - 1), max_blocks = max_padded / bs;
  const int nbits = E > 1 ? 32 - __clz(E - 1) : 0;
  if (tid == 0) bad = 0;
  for (int i = tid; i < nc * E; i += kRouteThreads) cnt[i] = 0;
  for (int i = tid; i < max_padded; i += kRouteThreads) sorted[i] = pad;
  for (int i = tid; i < max_blocks; i += kRouteThreads) experts[i] = 0;
  int ex[kRouteQ];
  bool any_bad = false;
#pragma unroll
  for (int q = 0; q < kRouteQ; q++) {
    const int i = (wv + q * kRouteWaves) * 64 + lane;
    ex[q] = i < n ? ids[i] : -1;
    any_bad |= i < n && (ex[q] < 0 || ex[q] >= E);
  }
  __syncthreads();  // bad = 0 and cnt = 0 are visible
  if (any_bad) bad = 1;
  __syncthreads();
  if (bad) {
    if (tid == 0) {
      ntpp[0] = 0;
      g_device_error = UB_ERR_INDEX;
    }
    return;
  }
  // rank among equal experts earlier in the chunk; group leaders store counts
  int rank[kRouteQ];
  const uint64_t below = (1ull << lane) - 1;
#pragma unroll
  for (int q = 0; q < kRouteQ; q++) {
    const int c = wv + q * kRouteWaves;
    rank[q] = 0;
    if (c < nc) {  // wave-uniform
      const int e = ex[q];
      uint64_t m = __ballot(e >= 0);
      for (int b = 0; b < nbits; b++) {
        const bool bit = (e >> b) & 1;
        const uint64_t on = __ballot(bit);
        m &= bit ? on : ~on;
      }
      rank[q] = __popcll(m & below);
      if (e >= 0 && rank[q] == 0) cnt[c * E + e] = __popcll(m);
    }
  }
  __syncthreads();
  for (int idx = tid; idx < G * E; idx += kRouteThreads) {
    const int e = idx % E, g = idx / E;
    int s = 0;
    for (int c = g * CPG; c < min(nc, (g + 1) * CPG); c++) s += cnt[c * E + e];
    part[g * E + e] = s;
  }
  __syncthreads();
  for (int idx = tid; idx < G * E; idx += kRouteThreads) {
    const int e = idx % E, g = idx / E;
    int run = 0;
    for (int h = 0; h < g; h++) run += part[h * E + e];
    for (int c = g * CPG; c < min(nc, (g + 1) * CPG); c++) {
      const int v = cnt[c * E + e];
      cnt[c * E + e] = run;
      run += v;
    }
    if (g == G - 1) eoff[e + 1] = (run + bs - 1) / bs * bs;  // padded count, scanned below
  }
  __syncthreads();
  if (tid < 64) {  // inclusive scan of the padded counts, 64 at a time
    int carry = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + tid;
      int v = e < E ? eoff[e + 1] : 0;
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(v, o, 64);
        if (tid >= o) v += u;
      }
      if (e < E) eoff[e + 1] = carry + v;
      carry += __shfl(v, 63, 64);
    }
    if (tid == 0) eoff[0] = 0;
  }
  __syncthreads();
  const int total = eoff[E];
#pragma unroll
  for (int q = 0; q < kRouteQ; q++) {
    const int c = wv + q * kRouteWaves;
    if (c < nc && ex[q] >= 0) sorted[eoff[ex[q]] + cnt[c * E + ex[q]] + rank[q]] = c * 64 + lane;
  }
  for (int b = tid; b < total / bs; b += kRouteThreads) {
    int lo = 0, hi = E;  // last e with eoff[e] <= b*bs
    const int v = b * bs;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (eoff[mid] <= v) lo = mid; else hi = mid;
    }
    experts[b] = lo;
  }
  if (tid == 0) ntpp[0] = total;
}

__global__ void __launch_bounds__(kRouteThreads) k_moe_align_small(
    const int* __restrict__ ids, int* __restrict__ sorted, int* __restrict__ experts,
    int* __restrict__ ntpp, int n, int E, int bs) {
  extern __shared__ int sh[];
  align_small_body(ids, sh, sorted, experts, ntpp, n, E, bs);
}

size_t align_small_lds(int n, int E) {
  const int nc = (n + 63) / 64;
  const int G = std::max(1, std::min(nc, kRouteThreads / E));
  return sizeof(int) * ((size_t)nc * E + (size_t)G * E + E + 2);
}

bool align_small_ok(int n, int E) { return n > 0 && n <= kRouteMaxN && align_small_lds(n, E) <= 96 * 1024; }
void align_small_launch(const int* ids, int* sorted, int* experts, int* ntpp, int n, int E, int bs,
                        hipStream_t s) {
  const size_t lds = align_small_lds(n, E);
  (void)hipFuncSetAttribute((const void*)k_moe_align_small, hipFuncAttributeMaxDynamicSharedMemorySize,
                      (int)lds);
  k_moe_align_small<<<1, kRouteThreads, lds, s>>>(ids, sorted, experts, ntpp, n, E, bs);
}

// ======================================================== grouped expert GEMM
// C[s, n] = T(acc * (scale[e,n]) (+ bias[e,n]) (* topk_w[s])) with
//   acc = sum_k A[s / topk_str, k] * B[e, n, k],  B bf16/f16 or int8 [E, N, K]
// for every slot s of every sorted block with expert e != -1; e == -1 zeroes
// the block's rows.
//
// The expert weights are the traffic (each expert's [N, K] matrix is read
// once per sorted block of that expert, ~32 flop per weight byte), so the
// kernel is built to keep HBM streaming: block tile 32 rows (of the sorted
// block) x 32 NWV columns, NWV wavefronts along N (one 32 x 32 MFMA tile
// each).  The gathered A rows and the weight tile travel HBM -> LDS by
// direct-to-LDS loads through a ring of NS K-step stages of BK, so NS - 1
// K-steps of loads are in flight per workgroup; int8 weights stay int8 in
// LDS and are widened to T exactly (|q| <= 128) as MFMA operands.  Within a
// 32-k pair of MFMAs a lane feeds 16 k-consecutive values (the same k
// permutation on both operands leaves the dot unchanged), so every fragment
// is one or two 16-byte LDS reads; both tiles are XOR-swizzled in 16-byte
// units against bank conflicts.
constexpr int MBM = 32;  // rows of a sorted block per workgroup

struct MoeArgs {
  void* C;
  const void* A;
  const void* B;
  const void* Bs;   // int8 path: per-channel scales T [E, N]
  const void* bias; // T [E, N] or null
  const float* tw;  // [topk_ids_size] or null
  const int* sorted;
  const int* eids;
  const int* ntpp;
  int K, N, E, tis, top_k, bs, mrw;
  int act;  // 1: gated SiLU output C[s, n] = T(silu(g) u), g / u = weight rows n / N/2 + n
  int a_div;  // slot s reads A row s / a_div
};

template <int DT>
__device__ __forceinline__ f32x16 mfma(const uint4& a, const uint4& b, const f32x16& c) {
  if constexpr (DT == UB_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// 8 int8 (two dwords) -> 8 T holding q + 128 (exact: 0..255 fit T's
// significand); the caller subtracts 128 * (sum of the A row) after the
// dot.  1.75 VALU ops per value: one xor per 4, a byte convert each, one
// pack per 2.
template <int DT>
__device__ __forceinline__ uint4 i8x8_to_t_off(uint32_t lo, uint32_t hi) {
  typedef unsigned char u8x4 __attribute__((ext_vector_type(4)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  const u8x4 L = __builtin_bit_cast(u8x4, lo ^ 0x80808080u), H = __builtin_bit_cast(u8x4, hi ^ 0x80808080u);
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const u8x4& V = i < 2 ? L : H;
    const f32x2 f = {(float)V[2 * (i & 1)], (float)V[2 * (i & 1) + 1]};
    if constexpr (DT == UB_BF16) {
      typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
      o[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
    } else {
      typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
      o[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2));
    }
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}
// acc + the sum of the 8 T values of an MFMA fragment (f32, by v_dot2)
template <int DT>
__device__ __forceinline__ float frag_sum(const uint4& a, float acc) {
  const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    if constexpr (DT == UB_BF16) {
      typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
      const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
      acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w[i]), one, acc, false);
    } else {
      typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
      const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w[i]), one, acc, false);
    }
  }
  return acc;
}

// s_waitcnt vmcnt(n) for a wave-uniform runtime n (clamped to 15: waiting
// for more loads than needed is always safe).
__device__ __forceinline__ void wait_vm_le(int n) {
  switch (n < 0 ? 0 : n) {
#define UB_VM_CASE(i) case i: ub_wait_vmcnt<i>(); break;
    UB_VM_CASE(0) UB_VM_CASE(1) UB_VM_CASE(2) UB_VM_CASE(3) UB_VM_CASE(4) UB_VM_CASE(5)
    UB_VM_CASE(6) UB_VM_CASE(7) UB_VM_CASE(8) UB_VM_CASE(9) UB_VM_CASE(10) UB_VM_CASE(11)
    UB_VM_CASE(12) UB_VM_CASE(13) UB_VM_CASE(14)
#undef UB_VM_CASE
    default: ub_wait_vmcnt<15>(); break;
  }
}

template <int DT, bool Q8, int NWV, int BK, int NS>
__global__ void __launch_bounds__(64 * NWV) k_moe_gemm(MoeArgs a) {
  constexpr int BN = 32 * NWV;                        // columns per workgroup
  constexpr int WB = Q8 ? 1 : 2;                      // weight bytes per value
  constexpr int RA = BK * 2, UA = BK / 8;             // A row bytes / 16-byte units
  constexpr int RB = BK * WB, UB = RB / 16;           // weight row bytes / units
  constexpr int AB = MBM * RA;                        // A bytes per stage
  constexpr int BB = BN * RB;                         // weight bytes per stage
  constexpr int STB = AB + BB;
  constexpr int NAT = AB / 1024, NBT = BB / 1024;     // 1 KiB load instructions per stage
  static_assert(BK % 32 == 0 && NBT % NWV == 0, "tile shape");
  constexpr int NB = NBT / NWV;                       // weight loads per wave and stage
  constexpr int NAW = (NAT + NWV - 1) / NWV;          // A loads per wave (upper bound)
  // Bank swizzle: 16-byte unit u of tile row r is stored at unit u ^ sw(r),
  // sw(r) = (r / rows per 256-byte bank window) % units per row, so the 16
  // rows one ds_read_b128 pass touches land in distinct banks.
  constexpr int RPWA = RA >= 256 ? 1 : 256 / RA, RPWB = RB >= 256 ? 1 : 256 / RB;
  auto swa = [](int r) { return (r / RPWA) % UA; };
  auto swb = [](int r) { return (r / RPWB) % UB; };
  __shared__ __attribute__((aligned(16))) uint8_t smem[NS * STB];
  __shared__ __attribute__((aligned(16))) int srow[256];  // the block's row slots (32 used)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int blk = blockIdx.y, sub = blockIdx.z * MBM;
  // Output columns: BN per workgroup, or with act BN / 2, whose gate rows
  // (first half of the tile) and up rows (second half) are both loaded.
  const int NO = a.act ? a.N / 2 : a.N, CT = a.act ? BN / 2 : BN;
  const int n0 = blockIdx.x * CT;
  // weight row of tile row r (0 <= r < BN), valid when its output column is
  auto wrow_of = [&](int r) -> int { return a.act && r >= CT ? NO + n0 + r - CT : n0 + r; };
  auto ocol_of = [&](int r) -> int { return a.act && r >= CT ? n0 + r - CT : n0 + r; };
  // ntpp and the block's expert are read together (blk < the grid's
  // max_blocks, the experts_ids array's size)
  const int npad = *a.ntpp;
  const int e = a.eids[blk];
  if (blk * a.bs >= npad || sub >= a.bs) return;
  uint16_t* C = (uint16_t*)a.C;
  const int topk_str = a.a_div;
  const int K = a.K, N = a.N;
  const uint32_t sbase = ub_lds_addr(smem);
  // The block's row slots go to LDS first: by one 16-byte DMA per lane 0..7
  // of wave 0 when the block's first entry is 16-byte aligned (bs % 4 == 0),
  // so that no wait for them drains the weight loads issued next (vector
  // loads into registers would make the compiler wait for every load in
  // flight); by plain loads otherwise.
  const bool dma_rows = (a.bs & 3) == 0;
  if (dma_rows) {
    if (wave == 0) {
      const ub_u32x4 rs = ub_desc(a.sorted, (uint64_t)(a.tis + a.E * (a.bs - 1)) * 4);
      ub_lds_load16_at(rs, ub_lds_addr(srow), lane < 8 ? (uint32_t)lane * 16 : kDmaOOB,
                       (uint32_t)(blk * a.bs + sub) * 4);
    }
  } else if (tid < MBM) {
    const int rr = sub + tid;
    srow[tid] = rr < a.bs ? a.sorted[blk * a.bs + rr] : -1;
  }
  // sorted slot of row r of this block, or -1 for padding / rows past the block
  auto slot = [&](int r) -> int {
    const int s = sub + r < a.bs ? srow[r] : -1;
    return (s >= 0 && s < a.tis) ? s : -1;
  };
  if (e < 0 || e >= a.E) {
    if (wave == 0 && dma_rows) ub_wait_vmcnt<0>();
    __syncthreads();
    if (e == -1) {  // expert handled elsewhere (expert parallel): zero the rows
      for (int i = tid; i < MBM * CT; i += 64 * NWV) {
        const int r = i / CT, n = n0 + i % CT, s = slot(r);
        if (s >= 0 && n < NO) C[(size_t)s * NO + n] = 0;
      }
    } else if (tid == 0) {
      g_device_error = UB_ERR_INDEX;
    }
    return;
  }
  const int arows = (a.tis + a.a_div - 1) / a.a_div;
  const ub_u32x4 ra = ub_desc(a.A, (uint64_t)arows * K * 2);
  const uint64_t brow = (uint64_t)K * WB;
  const ub_u32x4 rb = ub_desc((const uint8_t*)a.B + (size_t)e * N * brow, (uint64_t)N * brow);

  // Per-lane offsets of this wave's loads at K-step 0.  Instruction i of a
  // stage covers 16-byte units [64 i, 64 i + 64) of its tile and goes to wave
  // i % NWV.  k beyond K reads zero: the check is against the row, so
  // K % BK != 0 is handled.
  uint32_t voA[NAW], voB[NB];
  int kA[NAW], kB[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const int p = (j * NWV + wave) * 64 + lane;
    const int r = p / UB, u = p % UB;
    const int c = u ^ swb(r);
    kB[j] = Q8 ? 16 * c : 8 * c;
    voB[j] = ocol_of(r) < NO ? (uint32_t)((size_t)wrow_of(r) * brow + 16 * c) : kDmaOOB;
  }
  // A instruction j of this wave is issued only if its first row is a real
  // slot: a block's real slots come first, padding fills the rest (on
  // average half of a 32-row block at the Qwen3-MoE shape).
  bool a_on[NAW];
  int nA = 0, nl = NB;  // this wave's A loads / all loads per stage (set once the rows are known)
  auto issue_a = [&](int kt, uint32_t st) {
    const int k0 = kt * BK;
#pragma unroll
    for (int j = 0; j < NAW; j++)
      if (a_on[j])
        ub_lds_load16_at(ra, st + (j * NWV + wave) * 1024, k0 + kA[j] < K ? voA[j] : kDmaOOB,
                         (uint32_t)k0 * 2);
  };
  auto issue_w = [&](int kt, uint32_t st) {
    const int k0 = kt * BK;
#pragma unroll
    for (int j = 0; j < NB; j++)
      ub_lds_load16_at(rb, st + AB + (j * NWV + wave) * 1024, k0 + kB[j] < K ? voB[j] : kDmaOOB,
                       (uint32_t)k0 * WB);
  };

  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; r++) acc[r] = 0.f;
  float rsum = 0.f;  // int8 path: sum of this lane's A row over its k half
  const int l32 = lane & 31, kh = lane >> 5;
  const int bcol = wave * 32 + l32;
  const int nk = (K + BK - 1) / BK;
  const int P = min(NS - 1, nk);  // prologue stages
  // prologue: weights first (they need only the expert), then the row slots
  // are waited for and the gathered A rows issued
#pragma unroll
  for (int j = 0; j < NS - 1; j++)
    if (j < nk) issue_w(j, sbase + j * STB);
  if (wave == 0 && dma_rows) wait_vm_le(NB * P);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): plain row stores
  ub_barrier();
  const int nreal = __popcll(__ballot(lane < MBM && slot(lane) >= 0));  // real rows: 0 .. nreal-1
#pragma unroll
  for (int j = 0; j < NAW; j++) {
    const int i = j * NWV + wave;
    kA[j] = 1 << 30;
    voA[j] = kDmaOOB;
    a_on[j] = i < NAT && i * 64 / UA < nreal;
    nA += a_on[j] ? 1 : 0;
    if (i < NAT) {
      const int p = i * 64 + lane;
      const int r = p / UA, c = (p % UA) ^ swa(r);
      const int sr = slot(r);
      kA[j] = 8 * c;
      voA[j] = sr >= 0 ? (uint32_t)(((size_t)(sr / topk_str) * K + 8 * c) * 2) : kDmaOOB;
    }
  }
  nl = nA + NB;
#pragma unroll
  for (int j = 0; j < NS - 1; j++)
    if (j < nk) issue_a(j, sbase + j * STB);
  for (int kt = 0; kt < nk; kt++) {
    const uint32_t st = sbase + (kt % NS) * STB;
    // stage kt has landed once at most the loads issued after its A loads
    // are outstanding: the later prologue A loads and the stages issued in
    // the loop since
    const int later = kt < P ? (P - 1 - kt) * nA + max(0, min(kt, nk - (NS - 1))) * nl
                             : min(NS - 2, nk - 1 - kt) * nl;
    wait_vm_le(later);
    ub_barrier();  // stage kt visible; every wave is done with stage kt - 1
    if (kt + NS - 1 < nk) {
      issue_a(kt + NS - 1, sbase + ((kt + NS - 1) % NS) * STB);
      issue_w(kt + NS - 1, sbase + ((kt + NS - 1) % NS) * STB);
    }
    // pair sp: k = 32 sp + 16 kh .. +16 on both operands, two MFMAs
    uint4 af[BK / 16], bf[BK / 16];
#pragma unroll
    for (int sp = 0; sp < BK / 32; sp++) {
      const int c0 = 4 * sp + 2 * kh;  // A's 16-byte units (8 k each)
      af[2 * sp] = ub_lds_read16(st + l32 * RA + ((c0 ^ swa(l32)) << 4));
      af[2 * sp + 1] = ub_lds_read16(st + l32 * RA + (((c0 + 1) ^ swa(l32)) << 4));
      if constexpr (Q8) {
        const int u = 2 * sp + kh;  // 16 int8 k
        const uint4 w = ub_lds_read16(st + AB + bcol * RB + ((u ^ swb(bcol)) << 4));
        bf[2 * sp] = i8x8_to_t_off<DT>(w.x, w.y);
        bf[2 * sp + 1] = i8x8_to_t_off<DT>(w.z, w.w);
        rsum = frag_sum<DT>(af[2 * sp + 1], frag_sum<DT>(af[2 * sp], rsum));
      } else {
        bf[2 * sp] = ub_lds_read16(st + AB + bcol * RB + ((c0 ^ swb(bcol)) << 4));
        bf[2 * sp + 1] = ub_lds_read16(st + AB + bcol * RB + (((c0 + 1) ^ swb(bcol)) << 4));
      }
    }
#pragma unroll
    for (int j = 0; j < BK / 16; j++) acc = mfma<DT>(af[j], bf[j], acc);
  }
  // int8 weights entered as q + 128: subtract 128 x (sum of the A row)
  // (gathered for every lane here: the cross-lane reads must not run under
  // the epilogue's divergent exits)
  float rrow[16];
  if constexpr (Q8) {
    rsum += __shfl_xor(rsum, 32);
#pragma unroll
    for (int r = 0; r < 16; r++) rrow[r] = __shfl(rsum, 8 * (r >> 2) + 4 * kh + (r & 3));
  }
  // epilogue: lane l, register r -> row 8(r/4) + 4(l/32) + r%4, tile column
  // wave*32 + l%32 (weight row wn, output column oc)
  const int wn = wrow_of(bcol), oc = ocol_of(bcol);
  const bool col_ok = oc < NO;
  float sc = 1.f, bv = 0.f;
  if (col_ok) {
    if constexpr (Q8) sc = tof<DT>(((const uint16_t*)a.Bs)[(size_t)e * N + wn]);
    if (a.bias) bv = tof<DT>(((const uint16_t*)a.bias)[(size_t)e * N + wn]);
  }
  uint16_t vt[16];
#pragma unroll
  for (int r = 0; r < 16; r++) {
    const int row = 8 * (r >> 2) + 4 * kh + (r & 3);
    const int s = slot(row);
    float v = acc[r];
    if constexpr (Q8) v = (v - 128.f * rrow[r]) * sc;
    if (a.bias) v = v + bv;
    if (!a.act && a.mrw && s >= 0) v = v * a.tw[s];
    vt[r] = fromf<DT>(v);
    if (!a.act && s >= 0 && col_ok) C[(size_t)s * N + oc] = vt[r];
  }
  if (!a.act) return;
  // Gated SiLU, as silu_and_mul on the T-rounded GEMM outputs: the up
  // wavefronts hand their T values to the gate wavefronts through LDS.
  __syncthreads();  // every wave is past its last read of the ring
  uint16_t* ex = (uint16_t*)smem;  // [MBM][CT]
  const bool up = bcol >= CT;
  if (up) {
#pragma unroll
    for (int r = 0; r < 16; r++) ex[(8 * (r >> 2) + 4 * kh + (r & 3)) * CT + bcol - CT] = vt[r];
  }
  __syncthreads();
  if (up || !col_ok) return;
#pragma unroll
  for (int r = 0; r < 16; r++) {
    const int row = 8 * (r >> 2) + 4 * kh + (r & 3);
    const int s = slot(row);
    if (s < 0) continue;
    const float g = tof<DT>(vt[r]), u = tof<DT>(ex[row * CT + bcol]);
    C[(size_t)s * NO + oc] = fromf<DT>(g / (1.f + expf(-g)) * u);
  }
}

// Variants (knob moe_gemm_path): 1: 128 columns, BK 128, 3 stages;
// 2: 256 columns, BK 64, 4 stages; 3: 128 columns, BK 64, 6 stages;
// 4: 256 columns, BK 128, 3 stages (int8 only); 5: 128 columns, BK 64,
// 4 stages; 6 / 7: 64 columns, BK 64, 4 / 6 stages; 8: 128 columns, BK 64,
// 3 stages; 9: 64 columns, BK 128, 3 stages.  Automatic (0): 1 for int8
// experts with K >= 1536 and for 16-bit experts, else 8 -- measured on
// MI355X at the Qwen3-MoE shapes (gate/up K = 2048, down K = 768), where
// both stream within ~2% of the same ring with the MFMA work removed.
// (Weights loaded straight into MFMA-operand registers measured slower:
// 32 lanes x 32 contiguous bytes per instruction streams ~17% below the
// 128-byte row runs of the direct-to-LDS loads.)
template <int DT, bool Q8>
void moe_gemm_launch(int path, const MoeArgs& a, int max_blocks, hipStream_t s) {
  auto go = [&](auto kern, int nwv) {
    dim3 grid(ub_cdiv(a.act ? a.N / 2 : a.N, a.act ? 16 * nwv : 32 * nwv), max_blocks,
              ub_cdiv(a.bs, MBM));
    kern<<<grid, 64 * nwv, 0, s>>>(a);
  };
  if (path == 0) path = !Q8 || a.K >= 1536 ? 1 : 8;
  switch (path) {
    case 2: go(k_moe_gemm<DT, Q8, 8, 64, 4>, 8); break;
    case 3: go(k_moe_gemm<DT, Q8, 4, 64, 6>, 4); break;
    case 4:  // 216 KiB of LDS with 16-bit weights: int8 only
      if constexpr (Q8) go(k_moe_gemm<DT, Q8, 8, 128, 3>, 8);
      else go(k_moe_gemm<DT, Q8, 4, 128, 3>, 4);
      break;
    case 5: go(k_moe_gemm<DT, Q8, 4, 64, 4>, 4); break;
    case 6: go(k_moe_gemm<DT, Q8, 2, 64, 4>, 2); break;
    case 7: go(k_moe_gemm<DT, Q8, 2, 64, 6>, 2); break;
    case 8: go(k_moe_gemm<DT, Q8, 4, 64, 3>, 4); break;
    case 9: go(k_moe_gemm<DT, Q8, 2, 128, 3>, 2); break;
    default: go(k_moe_gemm<DT, Q8, 4, 128, 3>, 4); break;
  }
}

int moe_gemm(const char* nm, int dt, bool q8, void* C, const void* A, const void* B,
             const void* Bscale, const void* bias, const float* tw, const int* sorted,
             const int* eids, const int* ntpp, int M, int K, int N, int E, int tis, int top_k,
             int bs, int mrw, int bias_flag, void* stream, int act = 0, int a_div = 0) {
  UB_REQUIRE(K > 0 && N > 0 && E > 0 && bs > 0 && tis >= 0 && top_k > 0,
             "%s: K=%d N=%d E=%d block_size=%d topk_ids_size=%d top_k=%d", nm, K, N, E, bs, tis,
             top_k);
  UB_REQUIRE(K % 32 == 0, "%s: K=%d must be a multiple of 32", nm, K);
  (void)M;
  if (tis == 0) return UB_OK;
  UB_REQUIRE(C && A && B && sorted && eids && ntpp, "%s: null pointer", nm);
  UB_REQUIRE(!mrw || tw, "%s: mul_routed_weight needs topk_weights", nm);
  UB_REQUIRE(!q8 || Bscale, "%s: int8 experts need scales", nm);
  UB_REQUIRE(!act || (N % 2 == 0 && !mrw), "%s: gated output needs an even N and no routed weight",
             nm);
  MoeArgs a{C, A, B, Bscale, bias_flag ? bias : nullptr, tw, sorted, eids, ntpp,
            K, N, E, tis, top_k, bs, mrw, act,
            // the reference's invoke_fused_moe reads one A row per slot when
            // the routed weight is applied (the down projection), one per
            // token otherwise; the status-returning GEMM always one per token
            a_div ? a_div : (mrw ? 1 : top_k)};
  const int max_blocks = (tis + E * (bs - 1)) / bs;
  hipStream_t s = ub_stream(stream);
  const int path = ub_tune(UB_TUNE_MOE_GEMM_PATH);
  if (dt == UB_BF16) {
    if (q8) moe_gemm_launch<UB_BF16, true>(path, a, max_blocks, s);
    else moe_gemm_launch<UB_BF16, false>(path, a, max_blocks, s);
  } else {
    if (q8) moe_gemm_launch<UB_F16, true>(path, a, max_blocks, s);
    else moe_gemm_launch<UB_F16, false>(path, a, max_blocks, s);
  }
  return ub_check_launch(nm);
}

// ========================================================= silu_and_mul / sum
// out[t, i] = T(silu(x[t, i]) * x[t, d + i]), silu(g) = g / (1 + exp(-g)).
template <int DT>
__global__ void __launch_bounds__(256) k_silu_and_mul(const uint16_t* __restrict__ x,
                                                      uint16_t* __restrict__ out, int T, int d) {
  const size_t n = (size_t)T * d;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t t = i / d, c = i % d;
    const float g = tof<DT>(x[t * 2 * d + c]), u = tof<DT>(x[t * 2 * d + d + c]);
    out[i] = fromf<DT>(g / (1.f + expf(-g)) * u);
  }
}
// out[t, n] = T(sum_j in[t*k + j, n]), f32 accumulation in slot order.
template <int DT>
__global__ void __launch_bounds__(256) k_moe_sum(const uint16_t* __restrict__ in,
                                                 uint16_t* __restrict__ out, int T, int k, int N) {
  const size_t n = (size_t)T * N;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t t = i / N, c = i % N;
    float s = 0.f;
    for (int j = 0; j < k; j++) s += tof<DT>(in[(t * k + j) * N + c]);
    out[i] = fromf<DT>(s);
  }
}
// The same for N % 8 == 0, eight columns per thread by 16-byte loads (the k
// loads of a thread are independent, so one round trip covers them).
template <int DT>
__global__ void __launch_bounds__(256) k_moe_sum8(const uint4* __restrict__ in,
                                                  uint4* __restrict__ out, int T, int k, int N8) {
  const size_t n = (size_t)T * N8;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t t = i / N8, c = i % N8;
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < k; j++) {
      const uint4 v = in[(t * k + j) * N8 + c];
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; q++) {
        s[2 * q] += tof<DT>((uint16_t)(w[q] & 0xffff));
        s[2 * q + 1] += tof<DT>((uint16_t)(w[q] >> 16));
      }
    }
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; q++) o[q] = (uint32_t)fromf<DT>(s[2 * q]) | ((uint32_t)fromf<DT>(s[2 * q + 1]) << 16);
    out[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// ============================================================ legacy moe ops
// moe_{f16,bf16} (moe_host.cpp:27-93): for each pair k with idx[k] < N:
// y[idx[k], :] = T(y + T(e_out[k, :] * w[idx[k]*topk + top[k]])) when
// top[k] < topk.  The reference runs the pairs on 24 cores with unguarded
// read-modify-writes of y; here each column walks the pairs in order, so
// repeated rows accumulate deterministically.
template <int DT>
__global__ void __launch_bounds__(256) k_moe_combine(uint16_t* __restrict__ y,
                                                     const uint16_t* __restrict__ e_out,
                                                     const float* __restrict__ w,
                                                     const uint32_t* __restrict__ idx,
                                                     const uint32_t* __restrict__ top, int N,
                                                     int K, int M, int topk) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= M) return;
  for (int kk = 0; kk < K; kk++) {
    const uint32_t r = idx[kk], tp = top[kk];
    if (r >= (uint32_t)N || tp >= (uint32_t)topk) continue;
    const float wv = w[(size_t)r * topk + tp];
    const uint16_t prod = fromf<DT>(tof<DT>(e_out[(size_t)kk * M + c]) * wv);
    y[(size_t)r * M + c] = fromf<DT>(tof<DT>(y[(size_t)r * M + c]) + tof<DT>(prod));
  }
}

// indexed_moe_{f16,bf16} (moe_host.cpp:118-293): out[b, i, :] =
// W[idx[b,i]] (N x K) . in[b, M == 1 ? 0 : i, :], summed in f32 with k in order
// and no fused multiply-add (the reference's CPU check moe_matmul,
// moe_host.cpp:325-355, gives the same bits); pairs whose
// expert id is >= num_experts are left untouched, as in the reference.
// One workgroup per (b, i); the input row is staged in LDS and each lane owns
// columns, reading 16 bytes of its weight row per step.
template <int DT>
__global__ void __launch_bounds__(256) k_indexed_moe(const uint16_t* __restrict__ in,
                                                     const uint16_t* __restrict__ w,
                                                     uint16_t* __restrict__ out,
                                                     const uint32_t* __restrict__ idx, int N,
                                                     int K, int M, int topk, int E) {
  extern __shared__ float xin[];
  const int pair = blockIdx.y, b = pair / topk, i = pair % topk;
  const uint32_t e = idx[pair];
  if (e >= (uint32_t)E) return;
  const uint16_t* xr = in + ((size_t)b * M + (M == 1 ? 0 : i)) * K;
  for (int k = threadIdx.x; k < K; k += blockDim.x) xin[k] = tof<DT>(xr[k]);
  __syncthreads();
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const uint16_t* wr = w + ((size_t)e * N + n) * K;
  float acc = 0.f;
  for (int k = 0; k < K; k += 8) {
    const uint4 v = *(const uint4*)(wr + k);
    const uint32_t ws[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      acc = __fadd_rn(acc, __fmul_rn(xin[k + 2 * j], tof<DT>((uint16_t)(ws[j] & 0xffff))));
      acc = __fadd_rn(acc, __fmul_rn(xin[k + 2 * j + 1], tof<DT>((uint16_t)(ws[j] >> 16))));
    }
  }
  out[((size_t)b * topk + i) * N + n] = fromf<DT>(acc);
}

int grid1(size_t n) { return (int)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536); }

}  // namespace

// ======================================================================= ABI
UB_API int ubridge_device_error(void* stream) {
  int v = 0;
  hipError_t e = hipStreamSynchronize(ub_stream(stream));
  if (e != hipSuccess) return ub_set_error(UB_ERR_LAUNCH, "sync: %s", hipGetErrorString(e));
  e = hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_device_error), sizeof(int));
  if (e != hipSuccess) return ub_set_error(UB_ERR_LAUNCH, "read device flag: %s", hipGetErrorString(e));
  if (v) {
    const int zero = 0;
    (void)hipMemcpyToSymbol(HIP_SYMBOL(g_device_error), &zero, sizeof(int));
    ub_set_error(v, "device-side index out of range (expert id / real_token_num)");
  }
  return v;
}

UB_API void topk_softmax_f32(const float* in, float* out, int* idx, int T, int E, int k, int norm,
                             void* stream) {
  topk_softmax_launch<UB_F32>(in, out, idx, T, E, k, norm, stream, "topk_softmax_f32");
}
UB_API void topk_softmax_f16(const void* in, void* out, int* idx, int T, int E, int k, int norm,
                             void* stream) {
  topk_softmax_launch<UB_F16>(in, out, idx, T, E, k, norm, stream, "topk_softmax_f16");
}
UB_API void topk_softmax_bf16(const void* in, void* out, int* idx, int T, int E, int k, int norm,
                              void* stream) {
  topk_softmax_launch<UB_BF16>(in, out, idx, T, E, k, norm, stream, "topk_softmax_bf16");
}

// Routing for the grouped GEMM in one call: topk_softmax (T weights and ids,
// plus their f32 values for the GEMM's routed-weight operand) and
// moe_align_block_size, as two launches: the top-k over the whole GPU (one
// token per lane group) and the align in one workgroup.  (Both in one
// 1024-thread workgroup measured 2.5x slower at 256 tokens x 128 experts:
// the top-k needs the GPU's parallelism more than a launch is worth.)
static int moe_align_launch(int* sorted_ids, int* experts_ids, int* num_tokens_post_pad,
                            const int* topk_ids, const int* real_token_num,
                            const int* expert_map, int num_experts, int block_size,
                            int token_num, int topk, void* stream, const char* nm);

UB_API int ubridge_moe_route(const void* logits, int dtype, void* topk_w, float* topk_w_f32,
                             int* topk_ids, int* sorted_ids, int* experts_ids,
                             int* num_tokens_post_pad, int T, int E, int k, int renormalize,
                             int block_size, void* stream) {
  const char* nm = "ubridge_moe_route";
  UB_REQUIRE(T >= 0 && E > 0 && E <= 1024 && k > 0 && k <= E && k <= 64 && block_size > 0,
             "%s: T=%d E=%d k=%d block_size=%d", nm, T, E, k, block_size);
  UB_REQUIRE(dtype == UB_F32 || dtype == UB_F16 || dtype == UB_BF16, "%s: dtype %d", nm, dtype);
  UB_REQUIRE(logits && topk_w && topk_ids && sorted_ids && experts_ids && num_tokens_post_pad,
             "%s: null pointer", nm);
  int e = dtype == UB_F32   ? topk_softmax_launch<UB_F32>(logits, topk_w, topk_ids, T, E, k,
                                                         renormalize, stream, nm, topk_w_f32)
          : dtype == UB_F16 ? topk_softmax_launch<UB_F16>(logits, topk_w, topk_ids, T, E, k,
                                                         renormalize, stream, nm, topk_w_f32)
                            : topk_softmax_launch<UB_BF16>(logits, topk_w, topk_ids, T, E, k,
                                                          renormalize, stream, nm, topk_w_f32);
  if (e) return e;
  return moe_align_launch(sorted_ids, experts_ids, num_tokens_post_pad, topk_ids, nullptr,
                          nullptr, E, block_size, T, k, stream, nm);
}

static int moe_align_launch(int* sorted_ids, int* experts_ids, int* num_tokens_post_pad,
                            const int* topk_ids, const int* real_token_num,
                            const int* expert_map, int num_experts, int block_size,
                            int token_num, int topk, void* stream, const char* nm) {
  UB_REQUIRE(num_experts > 0 && num_experts <= 1024 && block_size > 0 && token_num >= 0 &&
                 topk > 0,
             "%s: num_experts=%d (<= 1024) block_size=%d token_num=%d topk=%d", nm, num_experts,
             block_size, token_num, topk);
  UB_REQUIRE(sorted_ids && experts_ids && num_tokens_post_pad && (topk_ids || token_num == 0),
             "%s: null pointer", nm);
  if (!real_token_num && !expert_map && align_small_ok(token_num * topk, num_experts)) {
    align_small_launch(topk_ids, sorted_ids, experts_ids, num_tokens_post_pad, token_num * topk,
                       num_experts, block_size, ub_stream(stream));
    return ub_check_launch(nm);
  }
  const size_t lds = sizeof(int) * ((size_t)(kAlignWaves + 1) * num_experts + 1);
  (void)hipFuncSetAttribute((const void*)k_moe_align, hipFuncAttributeMaxDynamicSharedMemorySize,
                      (int)lds);
  k_moe_align<<<1, kAlignThreads, lds, ub_stream(stream)>>>(
      sorted_ids, experts_ids, num_tokens_post_pad, topk_ids, real_token_num, expert_map,
      num_experts, block_size, token_num, topk);
  return ub_check_launch(nm);
}

UB_API void moe_align_block_size(int* sorted_ids, int* experts_ids, int* num_tokens_post_pad,
                                 const int* topk_ids, const int* real_token_num,
                                 const int* expert_map, int num_experts, int block_size,
                                 int token_num, int topk, void* stream) {
  moe_align_launch(sorted_ids, experts_ids, num_tokens_post_pad, topk_ids, real_token_num,
                   expert_map, num_experts, block_size, token_num, topk, stream,
                   "moe_align_block_size");
}

UB_API void invoke_fused_moe_bf16(void* C, const void* A, const void* B, const void* bias,
                                  const float* topk_weights, const int* sorted_ids,
                                  const int* experts_ids, const int* num_tokens_post_pad, int M,
                                  int K, int N, int E, int topk_ids_size, int top_k,
                                  int block_size, int mul_routed_weight, int bias_flag,
                                  void* stream) {
  moe_gemm("invoke_fused_moe_bf16", UB_BF16, false, C, A, B, nullptr, bias, topk_weights,
           sorted_ids, experts_ids, num_tokens_post_pad, M, K, N, E, topk_ids_size, top_k,
           block_size, mul_routed_weight, bias_flag, stream);
}
UB_API void invoke_fused_moe_f16(void* C, const void* A, const void* B, const void* bias,
                                 const float* topk_weights, const int* sorted_ids,
                                 const int* experts_ids, const int* num_tokens_post_pad, int M,
                                 int K, int N, int E, int topk_ids_size, int top_k,
                                 int block_size, int mul_routed_weight, int bias_flag,
                                 void* stream) {
  moe_gemm("invoke_fused_moe_f16", UB_F16, false, C, A, B, nullptr, bias, topk_weights,
           sorted_ids, experts_ids, num_tokens_post_pad, M, K, N, E, topk_ids_size, top_k,
           block_size, mul_routed_weight, bias_flag, stream);
}
// W8A16 experts: B int8 [E, N, K], B_scale T [E, N] per output channel.
UB_API int ubridge_fused_moe_w8a16(void* C, const void* A, const int8_t* B, const void* B_scale,
                                   const void* bias, const float* topk_weights,
                                   const int* sorted_ids, const int* experts_ids,
                                   const int* num_tokens_post_pad, int M, int K, int N, int E,
                                   int topk_ids_size, int top_k, int block_size,
                                   int mul_routed_weight, int bias_flag, int dtype,
                                   void* stream) {
  const char* nm = "ubridge_fused_moe_w8a16";
  UB_REQUIRE(dtype == UB_BF16 || dtype == UB_F16, "%s: dtype %d", nm, dtype);
  return moe_gemm(nm, dtype, true, C, A, B, B_scale, bias, topk_weights, sorted_ids, experts_ids,
                  num_tokens_post_pad, M, K, N, E, topk_ids_size, top_k, block_size,
                  mul_routed_weight, bias_flag, stream);
}

int moe_sum_launch(void* out, const void* in, int T, int k, int N, int dtype, hipStream_t s);

// The down expert GEMM and the top-k combine in one call: C as
// ubridge_fused_moe_w8a16 writes it, then Y [topk_ids_size / top_k, N] =
// T(sum_j C[t top_k + j, :]) in slot order (ubridge_moe_sum's bits).  Two
// launches: a combine inside the GEMM's epilogue has to make each
// workgroup's rows visible to workgroups on other XCDs, a device-scope
// release that writes back the XCD's L2 per workgroup; measured at the
// Qwen3-MoE shape that made the down GEMM 10x slower than the separate sum.
UB_API int ubridge_fused_moe_w8a16_combine(void* Y, void* C, const void* A, const int8_t* B,
                                           const void* B_scale, const void* bias,
                                           const float* topk_weights, const int* sorted_ids,
                                           const int* experts_ids, const int* num_tokens_post_pad,
                                           int M, int K, int N, int E, int topk_ids_size,
                                           int top_k, int block_size, int mul_routed_weight,
                                           int bias_flag, int dtype, void* stream) {
  const char* nm = "ubridge_fused_moe_w8a16_combine";
  UB_REQUIRE(dtype == UB_BF16 || dtype == UB_F16, "%s: dtype %d", nm, dtype);
  UB_REQUIRE(top_k > 0 && topk_ids_size >= 0 && topk_ids_size % top_k == 0,
             "%s: topk_ids_size %d is not a multiple of top_k %d", nm, topk_ids_size, top_k);
  UB_REQUIRE(Y || topk_ids_size == 0, "%s: null pointer", nm);
  const int e = moe_gemm(nm, dtype, true, C, A, B, B_scale, bias, topk_weights, sorted_ids,
                         experts_ids, num_tokens_post_pad, M, K, N, E, topk_ids_size, top_k,
                         block_size, mul_routed_weight, bias_flag, stream);
  if (e) return e;
  return moe_sum_launch(Y, C, topk_ids_size / top_k, top_k, N, dtype, ub_stream(stream));
}

// The gate/up expert GEMM with silu_and_mul fused into its epilogue:
// C[s, n] = T(silu(g) * u), g and u the T-rounded outputs of weight rows n and
// N/2 + n, exactly what ubridge_fused_moe_w8a16 followed by silu_and_mul
// produce; C is [topk_ids_size, N/2].  No routed weight.
UB_API int ubridge_fused_moe_w8a16_silu(void* C, const void* A, const int8_t* B, const void* B_scale,
                                        const void* bias, const int* sorted_ids,
                                        const int* experts_ids, const int* num_tokens_post_pad,
                                        int M, int K, int N, int E, int topk_ids_size, int top_k,
                                        int block_size, int bias_flag, int dtype, void* stream) {
  const char* nm = "ubridge_fused_moe_w8a16_silu";
  UB_REQUIRE(dtype == UB_BF16 || dtype == UB_F16, "%s: dtype %d", nm, dtype);
  return moe_gemm(nm, dtype, true, C, A, B, B_scale, bias, nullptr, sorted_ids, experts_ids,
                  num_tokens_post_pad, M, K, N, E, topk_ids_size, top_k, block_size, 0, bias_flag,
                  stream, 1);
}

UB_API int ubridge_silu_and_mul(void* out, const void* x, int T, int d, int dtype, void* stream) {
  UB_REQUIRE(T >= 0 && d >= 0 && (dtype == UB_BF16 || dtype == UB_F16), "ubridge_silu_and_mul: args");
  if ((size_t)T * d == 0) return UB_OK;
  UB_REQUIRE(out && x, "ubridge_silu_and_mul: null pointer");
  hipStream_t s = ub_stream(stream);
  if (dtype == UB_BF16)
    k_silu_and_mul<UB_BF16><<<grid1((size_t)T * d), 256, 0, s>>>((const uint16_t*)x, (uint16_t*)out, T, d);
  else
    k_silu_and_mul<UB_F16><<<grid1((size_t)T * d), 256, 0, s>>>((const uint16_t*)x, (uint16_t*)out, T, d);
  return ub_check_launch("ubridge_silu_and_mul");
}

int moe_sum_launch(void* out, const void* in, int T, int k, int N, int dtype, hipStream_t s) {
  UB_REQUIRE(T >= 0 && k > 0 && N >= 0 && (dtype == UB_BF16 || dtype == UB_F16), "ubridge_moe_sum: args");
  if ((size_t)T * N == 0) return UB_OK;
  UB_REQUIRE(out && in, "ubridge_moe_sum: null pointer");
  if (N % 8 == 0 && ((uintptr_t)in & 15) == 0 && ((uintptr_t)out & 15) == 0) {
    if (dtype == UB_BF16)
      k_moe_sum8<UB_BF16><<<grid1((size_t)T * N / 8), 256, 0, s>>>((const uint4*)in, (uint4*)out, T, k, N / 8);
    else
      k_moe_sum8<UB_F16><<<grid1((size_t)T * N / 8), 256, 0, s>>>((const uint4*)in, (uint4*)out, T, k, N / 8);
  } else if (dtype == UB_BF16) {
    k_moe_sum<UB_BF16><<<grid1((size_t)T * N), 256, 0, s>>>((const uint16_t*)in, (uint16_t*)out, T, k, N);
  } else {
    k_moe_sum<UB_F16><<<grid1((size_t)T * N), 256, 0, s>>>((const uint16_t*)in, (uint16_t*)out, T, k, N);
  }
  return ub_check_launch("ubridge_moe_sum");
}
UB_API int ubridge_moe_sum(void* out, const void* in, int T, int k, int N, int dtype, void* stream) {
  return moe_sum_launch(out, in, T, k, N, dtype, ub_stream(stream));
}

#define UB_MOE_LEGACY(T, DT)                                                                     \
  UB_API void moe_##T(void* y, const void* e_out, const float* w, const uint32_t* idx,          \
                      const uint32_t* top, int N, int K, int M, int topk, void* stream) {        \
    UB_REQUIRE_V(N >= 0 && K >= 0 && M >= 0 && topk > 0, "moe_" #T ": args");                    \
    if ((size_t)K * M == 0) return;                                                              \
    UB_REQUIRE_V(y && e_out && w && idx && top, "moe_" #T ": null pointer");                     \
    k_moe_combine<DT><<<ub_cdiv(M, 256), 256, 0, ub_stream(stream)>>>(                           \
        (uint16_t*)y, (const uint16_t*)e_out, w, idx, top, N, K, M, topk);                       \
    ub_check_launch("moe_" #T);                                                                  \
  }                                                                                              \
  UB_API void indexed_moe_##T(const void* in, const void* w, void* out, const uint32_t* idx,    \
                              int N, int K, int M, int batch, int topk, int num_experts,         \
                              void* stream) {                                                    \
    UB_REQUIRE_V(N >= 0 && K >= 0 && K % 8 == 0 && M >= 1 && batch >= 0 && topk > 0,             \
                 "indexed_moe_" #T ": N=%d K=%d (multiple of 8) M=%d", N, K, M);                 \
    if ((size_t)batch * N == 0) return;                                                          \
    UB_REQUIRE_V(in && w && out && idx, "indexed_moe_" #T ": null pointer");                     \
    dim3 grid(ub_cdiv(N, 256), batch * topk);                                                    \
    k_indexed_moe<DT><<<grid, 256, (size_t)K * sizeof(float), ub_stream(stream)>>>(              \
        (const uint16_t*)in, (const uint16_t*)w, (uint16_t*)out, idx, N, K, M, topk,             \
        num_experts);                                                                            \
    ub_check_launch("indexed_moe_" #T);                                                          \
  }
UB_MOE_LEGACY(f16, UB_F16)
UB_MOE_LEGACY(bf16, UB_BF16)
#undef UB_MOE_LEGACY

// ================================================= status-returning MoE names
// The reference's graph-safe MoE trio (kernels/topsaten_moe_wrapper.cpp:80-
// 208, bound in src/ffi.rs:671-715) with the same arguments, each returning
// 0 on success or the error code ubridge_last_error would report.  They run
// the kernels above; none of them allocates, so each is capturable.

// topk_softmax_f32 plus token_expert_indices[t, j] = j * num_tokens + t (the
// source row of slot (t, j) in a top-k-major layout), written by the same
// launch.  norm_topk_prob renormalises the k weights to sum 1.
UB_API int topsaten_topk_softmax_f32(float* gating_output, float* topk_weights,
                                     int32_t* topk_indices, int32_t* token_expert_indices,
                                     int32_t num_tokens, int32_t num_experts, int32_t topk,
                                     int32_t norm_topk_prob, void* stream) {
  const char* nm = "topsaten_topk_softmax_f32";
  UB_REQUIRE((int64_t)num_tokens * topk <= INT32_MAX, "%s: num_tokens * topk overflows", nm);
  UB_REQUIRE(token_expert_indices || num_tokens == 0, "%s: null token_expert_indices", nm);
  return topk_softmax_launch<UB_F32>(gating_output, topk_weights, topk_indices, num_tokens,
                                     num_experts, topk, norm_topk_prob, stream, nm, nullptr,
                                     token_expert_indices);
}

// moe_align_block_size over topk_ids [num_tokens, topk] without an expert map
// or a device-side token count; sorted_token_ids holds num_tokens * topk +
// num_experts * (block_size - 1) slots and experts_ids that / block_size.
UB_API int topsaten_moe_align_block_size(int32_t* sorted_token_ids, int32_t* experts_ids,
                                         int32_t* num_tokens_post_pad, int32_t* topk_ids,
                                         int32_t num_tokens, int32_t topk, int32_t num_experts,
                                         int32_t block_size, void* stream) {
  return moe_align_launch(sorted_token_ids, experts_ids, num_tokens_post_pad, topk_ids, nullptr,
                          nullptr, num_experts, block_size, num_tokens, topk, stream,
                          "topsaten_moe_align_block_size");
}

// The grouped expert GEMM: C [num_tokens, topk, inter_dim] = A [num_tokens,
// hidden_dim] . B [num_experts, inter_dim, hidden_dim]^T per routed slot,
// times the slot's f32 weight when mul_routed_weight; slot t * topk + j
// reads A row t with or without the weight (unlike invoke_fused_moe, whose
// weighted form reads one A row per slot).  dtype_code is the
// reference's: 4 fp16, 5 bf16 (8, fp32, is not supported here: error 3).
// topk_ids is part of the reference's signature and not read: the slots come
// from sorted_token_ids.
UB_API int topsaten_fused_moe_gemm(void* c_ptr, void* a_ptr, void* b_ptr, float* topk_weights,
                                   int32_t* topk_ids, int32_t* sorted_token_ids,
                                   int32_t* expert_ids, int32_t* num_tokens_post_padded,
                                   int32_t mul_routed_weight, int32_t topk_val,
                                   int32_t block_size, int32_t num_tokens, int32_t hidden_dim,
                                   int32_t inter_dim, int32_t num_experts, int32_t dtype_code,
                                   void* stream) {
  const char* nm = "topsaten_fused_moe_gemm";
  (void)topk_ids;
  if (dtype_code != 4 && dtype_code != 5)
    return ub_set_error(UB_ERR_UNSUPPORTED, "%s: dtype_code %d (4 fp16, 5 bf16)", nm,
                        dtype_code);
  UB_REQUIRE(num_tokens >= 0 && (int64_t)num_tokens * topk_val <= INT32_MAX,
             "%s: num_tokens=%d topk=%d", nm, num_tokens, topk_val);
  return moe_gemm(nm, dtype_code == 4 ? UB_F16 : UB_BF16, false, c_ptr, a_ptr, b_ptr, nullptr,
                  nullptr, topk_weights, sorted_token_ids, expert_ids, num_tokens_post_padded,
                  num_tokens, hidden_dim, inter_dim, num_experts, num_tokens * topk_val,
                  topk_val, block_size, mul_routed_weight, 0, stream, 0, topk_val);
}

// The reference's release hook for capture-time workspaces
// (topsaten_moe_wrapper.cpp:214-216).  The three calls above use none; the
// hook frees the stream's library scratch pool (the slab and K-split
// buffers of the GEMM routes).
UB_API int ubridge_release_workspace(void* stream);
UB_API void topsaten_release_graph_workspace_pool(void* stream) {
  (void)ubridge_release_workspace(stream);
}
