// runtime.cpp -- sticky error state and library identity for libubridge_hip.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>

#include "common.h"

namespace {
thread_local int g_err = UB_OK;
thread_local char g_msg[512] = {0};
}  // namespace

int ub_set_error(int code, const char* fmt, ...) {
  g_err = code;
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
  return code;
}

int ub_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return ub_set_error(UB_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return UB_OK;
}

UB_API int ubridge_last_error(void) {
  int e = g_err;
  g_err = UB_OK;
  return e;
}

UB_API const char* ubridge_last_error_string(void) { return g_msg; }

UB_API const char* ubridge_version(void) { return "ubridge_amd 0.1 gfx950"; }

// ------------------------------------------------------- launch-shape knobs
// The reference picks GEMM tilings on the host from the problem shape
// (gemm_tuner.rs:326-600, GEMM_OP_PARAS :222-258, cached per shape).  Here
// each launcher applies its own shape rule; these knobs override a rule
// process-wide (0 = automatic), for tuning sweeps and for callers that
// know better.  Initial values come from the environment.
namespace {
struct Knob {
  const char* name;
  const char* env;
};
constexpr Knob kKnobs[UB_TUNE_COUNT] = {
    {"gemv_lds_rows", "UBRIDGE_GEMV_LDS"}, {"gemv_lds_waves", "UBRIDGE_GEMV_W"},
    {"gemv_rows", "UBRIDGE_GEMV_R"},       {"gemv_iters", "UBRIDGE_GEMV_U"},
    {"gemm_tile", "UBRIDGE_GEMM_TILE"},    {"gemv_mfma_m", "UBRIDGE_GEMV_MFMA_M"},
    {"w4a16_path", "UBRIDGE_W4A16_PATH"},    {"moe_gemm_path", "UBRIDGE_MOE_GEMM_PATH"},
    {"gemv_mm", "UBRIDGE_GEMV_MM"},        {"gemv_persist", "UBRIDGE_GEMV_PERSIST"},
    {"gemv_q80_lds", "UBRIDGE_GEMV_Q80_LDS"},
};
std::atomic<int> g_knob[UB_TUNE_COUNT];
std::atomic<bool> g_knob_init[UB_TUNE_COUNT];

int knob_index(const char* name) {
  if (!name) return -1;
  for (int i = 0; i < UB_TUNE_COUNT; i++)
    if (strcmp(name, kKnobs[i].name) == 0) return i;
  return -1;
}
}  // namespace

int ub_tune(int k) {
  if (!g_knob_init[k].load(std::memory_order_acquire)) {
    const char* v = getenv(kKnobs[k].env);
    int expected = 0;
    g_knob[k].compare_exchange_strong(expected, v ? atoi(v) : 0);
    g_knob_init[k].store(true, std::memory_order_release);
  }
  return g_knob[k].load(std::memory_order_relaxed);
}

// Set a knob by name ("gemv_lds_rows", "gemv_lds_waves", "gemv_rows",
// "gemv_iters", "gemm_tile", "gemv_mfma_m", "w4a16_path", "moe_gemm_path",
// "gemv_mm", "gemv_persist", "gemv_q80_lds"); 0
// restores the
// automatic rule.
UB_API int ubridge_tune_set(const char* name, int value) {
  const int k = knob_index(name);
  if (k < 0) return ub_set_error(UB_ERR_INVALID_ARG, "ubridge_tune_set: unknown knob '%s'",
                                 name ? name : "(null)");
  g_knob[k].store(value, std::memory_order_relaxed);
  g_knob_init[k].store(true, std::memory_order_release);
  return UB_OK;
}

// Current value of a knob (0 = automatic); unknown names set error 1 and
// return 0.
UB_API int ubridge_tune_get(const char* name) {
  const int k = knob_index(name);
  if (k < 0) {
    ub_set_error(UB_ERR_INVALID_ARG, "ubridge_tune_get: unknown knob '%s'", name ? name : "(null)");
    return 0;
  }
  return ub_tune(k);
}

// ------------------------------------------------------ stream workspaces
// Device scratch for kernels that split work across workgroups and combine
// partial results in a second launch (the reference's entry points take no
// workspace argument).  One buffer per (device, stream), grown on demand;
// every buffer handed out stays allocated until the process ends (a graph
// captured with it keeps working), and none is allocated while the stream is
// being captured (the caller then takes its single-launch form).  Work that
// shares a stream's buffer is ordered by that stream.
#include <map>
#include <mutex>
#include <utility>
namespace {
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, std::pair<void*, size_t>> g_ws;
}  // namespace

void* ub_stream_workspace(hipStream_t s, size_t bytes) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lk(g_ws_mu);
  auto& e = g_ws[{dev, s}];
  if (e.second >= bytes) return e.first;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess || st != hipStreamCaptureStatusNone)
    return nullptr;
  // A smaller buffer is kept, not freed: queued work or a captured graph may
  // still use it.
  void* p = nullptr;
  const size_t sz = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
  if (hipMalloc(&p, sz) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  e = {p, sz};
  return p;
}
