// common.h -- shared device helpers and the host-side error state for the
// ubridge_amd HIP library (gfx950 / CDNA4 only).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>
#include "../../include/ubridge_hip.h"  // definitions below must match the public ABI

#define UB_API extern "C" __attribute__((visibility("default")))

// ---------------------------------------------------------------- errors --
// The reference's host libraries return void and trap on bad indices
// (moe_kernel_compat.h op_assert).  Here every entry point records a sticky
// error code + message instead; ubridge_last_error() reads and clears it.
enum {
  UB_OK = 0,
  UB_ERR_INVALID_ARG = 1,
  UB_ERR_LAUNCH = 2,
  UB_ERR_UNSUPPORTED = 3,
  UB_ERR_INDEX = 4,
};
int ub_set_error(int code, const char* fmt, ...);
int ub_check_launch(const char* what);

// Launch-shape knobs (runtime.cpp): 0 = the automatic shape rule of the
// launcher that reads it; set through ubridge_tune_set() or, at first use,
// the environment variable named in runtime.cpp.
enum UbTune {
  UB_TUNE_GEMV_LDS_ROWS = 0,  // Q4_K LDS GEMV rows per wavefront (< 0: LDS path off)
  UB_TUNE_GEMV_LDS_WAVES,     // Q4_K LDS GEMV wavefronts per workgroup (4 / 8)
  UB_TUNE_GEMV_ROWS,          // register-path GEMV rows per wavefront (1 / 2 / 4)
  UB_TUNE_GEMV_ITERS,         // register-path GEMV block-iterations per pass (1 / 2)
  UB_TUNE_GEMM_TILE,          // MFMA GEMM tile: 1 = 128x128, 2 = 128x256, 3 = 256x256
  UB_TUNE_GEMV_MFMA_M,        // fewest tokens for the int8-MFMA GEMV (Q8_0 / Q4_K; > 16: off)
  UB_TUNE_W4A16_PATH,         // W4/W8 GEMMs: 0 automatic, 1 generic MFMA core only, 2 no decode GEMV, 3 / 5 GPTQ tile variants
  UB_TUNE_MOE_GEMM_PATH,      // MoE expert GEMM tile / ring variant (0 automatic, 1..5)
  UB_TUNE_GEMV_MM,            // multi-token ring GEMV variant (0 automatic, < 0 off)
  UB_TUNE_GEMV_PERSIST,       // one-launch Q4_K GEMV: 0 automatic, < 0 one-shot grid, > 0 persistent
                              // (2: issue after the math, 3: rolling prefetch)
  UB_TUNE_GEMV_Q80_LDS,       // one-launch Q4_0 / Q8_0 GEMV: 0 automatic, < 0 register path, > 0 LDS path
  UB_TUNE_GEMV_FUSE_M,        // most tokens of the one-launch quantize + GEMV (0 automatic = 4; 1..4)
  UB_TUNE_COUNT
};
int ub_tune(int knob);
// Device scratch for one call's kernels on stream s: at least `bytes`, from
// the caller's allocator when one is registered (ubridge_set_workspace_
// allocator: taken at construction, handed back on s at destruction, so the
// object must outlive the launches that use it), else from the library's
// per-(device, stream) pool (ubridge_release_workspace frees it).  Works while
// s captures a graph (the allocation is made outside the capture), so the
// route a call takes never depends on whether an eager call came first;
// get() is null only when the allocation itself fails.
class UbScratch {
 public:
  UbScratch(hipStream_t s, size_t bytes);
  ~UbScratch();
  UbScratch(const UbScratch&) = delete;
  UbScratch& operator=(const UbScratch&) = delete;
  void* get() const { return p_; }

 private:
  void* p_ = nullptr;
  hipStream_t s_ = nullptr;
  bool caller_ = false;
};

// hipBLASLt's per-device set-up (blaslt.cpp), made at the first call on the
// device of an entry point that can route to hipBLASLt, outside captures.
void ub_blaslt_prepare(hipStream_t s);

// Runs a scope with the calling thread's stream-capture mode relaxed, so a
// library-internal allocation or plan creation made while the caller's
// stream captures a graph is legal and stays out of the graph.
class UbRelaxCapture {
 public:
  UbRelaxCapture() { (void)hipThreadExchangeStreamCaptureMode(&m_); }
  ~UbRelaxCapture() { (void)hipThreadExchangeStreamCaptureMode(&m_); }

 private:
  hipStreamCaptureMode m_ = hipStreamCaptureModeRelaxed;
};

#define UB_REQUIRE(cond, ...)                                   \
  do {                                                          \
    if (!(cond)) return ub_set_error(UB_ERR_INVALID_ARG, __VA_ARGS__); \
  } while (0)
#define UB_REQUIRE_V(cond, ...)                                 \
  do {                                                          \
    if (!(cond)) { ub_set_error(UB_ERR_INVALID_ARG, __VA_ARGS__); return; } \
  } while (0)

static inline hipStream_t ub_stream(const void* s) { return (hipStream_t)const_cast<void*>(s); }

// ------------------------------------------------------------- numerics --
// bf16 / f16 are carried as raw 16-bit patterns so every rounding is explicit.
__device__ __forceinline__ float ub_bf16_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}
// IEEE round-to-nearest-even, NaN kept quiet.
__device__ __forceinline__ uint16_t ub_f32_to_bf16(float f) {
  uint32_t x = __float_as_uint(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}
__device__ __forceinline__ float ub_f16_to_f32(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}

// 6-bit scale / min of sub-block s (0..7) from the 12 packed bytes
// (get_scale_min_k4, quant.cpp:356-363), bytes given as three dwords.
__device__ __forceinline__ void q4k_scale_min(int s, uint32_t s0, uint32_t s1, uint32_t s2,
                                              int& sc, int& mn) {
  // selects, not an indexed array: a lane-varying s must not send the bytes
  // through private memory
  auto byte = [&](int i) -> int {
    const uint32_t w = i < 4 ? s0 : i < 8 ? s1 : s2;
    return (int)((w >> (8 * (i & 3))) & 0xff);
  };
  if (s < 4) {
    sc = byte(s) & 63;
    mn = byte(s + 4) & 63;
  } else {
    sc = (byte(s + 4) & 0xF) | ((byte(s - 4) >> 6) << 4);
    mn = (byte(s + 4) >> 4) | ((byte(s) >> 6) << 4);
  }
}
__device__ __forceinline__ uint16_t ub_f32_to_f16(float f) {
  return __half_as_ushort(__float2half_rn(f));
}

enum { UB_F32 = 0, UB_F16 = 1, UB_BF16 = 2 };
// GGML type ids.
enum { UB_Q4_0 = 2, UB_Q8_0 = 8, UB_Q4_K = 12 };

template <int DT>
__device__ __forceinline__ void ub_store(void* p, size_t i, float v) {
  if constexpr (DT == UB_F32) ((float*)p)[i] = v;
  else if constexpr (DT == UB_F16) ((uint16_t*)p)[i] = ub_f32_to_f16(v);
  else ((uint16_t*)p)[i] = ub_f32_to_bf16(v);
}
template <int DT>
__device__ __forceinline__ float ub_load(const void* p, size_t i) {
  if constexpr (DT == UB_F32) return ((const float*)p)[i];
  else if constexpr (DT == UB_F16) return ub_f16_to_f32(((const uint16_t*)p)[i]);
  else return ub_bf16_to_f32(((const uint16_t*)p)[i]);
}

// Wavefront (64-lane) butterfly sum; every lane ends with the total.
__device__ __forceinline__ float ub_wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

static inline int ub_cdiv(long a, long b) { return (int)((a + b - 1) / b); }
