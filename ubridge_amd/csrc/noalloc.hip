// noalloc.hip -- allocation-free form of ubridge_qmatmul (no counterpart in
// the reference): the activation workspace comes from a static device array.
#include "common.h"

#include <mutex>

// ============================================= allocation-free QMatMul
// For callers that cannot allocate (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc): the activation workspace
// of ubridge_qmatmul lives in a file-scope device array instead of a caller
// buffer.  Each GPU holds its own copy for the life of the process.  The
// array's name is a host-side stand-in, so host code only ever uses the
// per-device address hipGetSymbolAddress returns.
namespace {
constexpr size_t kNoAllocScratch = 4u << 20;  // 4 MiB (M*K limits: ubridge_qmatmul_noalloc below)
__device__ __align__(256) uint8_t scratch[kNoAllocScratch];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // per-device address of `scratch`, null until looked up

// Address of this device's `scratch`, looked up once per device with that
// device current (the caller's current device is the one the stream is on).
int scratch_ptr(void** out, const char* nm) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return ub_set_error(UB_ERR_LAUNCH, "%s: hipGetDevice: %s", nm, hipGetErrorString(e));
  UB_REQUIRE(dev >= 0 && dev < kMaxDevices, "%s: device %d beyond %d", nm, dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return ub_set_error(UB_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch): %s", nm,
                          hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return UB_OK;
}
}  // namespace

// gemv.hip: ubridge_qmatmul restricted to the forms that allocate nothing
int ub_qmatmul(int qtype, const void* w, const void* x, int x_dtype, void* y, int y_dtype, int M,
               int N, int K, void* workspace, size_t ws_bytes, void* stream, bool may_alloc);
size_t ub_qmatmul_noalloc_ws(int qtype, int M, int K);

UB_API size_t ubridge_qmatmul_noalloc_max_workspace(void) { return kNoAllocScratch; }

// ubridge_qmatmul with the workspace taken from the device's static scratch
// array: no hipMalloc / hipFree / allocating library call (at prefill sizes
// the GEMMs that dequantize on chip, not the slab + hipBLASLt form, and
// without the K split over workgroups).  Sizes whose workspace on those
// routes (the quantized activations: M*K up to ~3.68M elements for Q4_K,
// ~3.36M for Q4_0 / Q8_0; from 64 / 40 tokens also room for a bf16 copy of
// x: M*K up to 2,097,152) exceeds the array are rejected (error 1).  Every call on one GPU shares the array; calls that overlap on
// one GPU (different streams, no ordering) race.  Nothing in the array needs
// to start at zero: the activation quantizer writes every byte the GEMV reads.
UB_API int ubridge_qmatmul_noalloc(int qtype, const void* w, const void* x, int x_dtype, void* y,
                                   int y_dtype, int M, int N, int K, void* stream) {
  const char* nm = "ubridge_qmatmul_noalloc";
  UB_REQUIRE(qtype == UB_Q4_0 || qtype == UB_Q8_0 || qtype == UB_Q4_K, "%s: unsupported qtype %d",
             nm, qtype);
  UB_REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative shape", nm);
  const size_t need = ub_qmatmul_noalloc_ws(qtype, M, K);
  UB_REQUIRE(need <= kNoAllocScratch,
             "%s: M=%d K=%d needs a %zu-byte workspace, above the %zu-byte static scratch", nm, M,
             K, need, kNoAllocScratch);
  void* ws = nullptr;
  int e = scratch_ptr(&ws, nm);
  if (e) return e;
  return ub_qmatmul(qtype, w, x, x_dtype, y, y_dtype, M, N, K, ws, kNoAllocScratch, stream, false);
}
