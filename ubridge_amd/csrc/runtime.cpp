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
    {"gemv_q80_lds", "UBRIDGE_GEMV_Q80_LDS"}, {"gemv_fuse_m", "UBRIDGE_GEMV_FUSE_M"},
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
// "gemv_mm", "gemv_persist", "gemv_q80_lds", "gemv_fuse_m"); 0
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

// ------------------------------------------------------ device scratch
// Scratch for kernels that split work across workgroups and combine partial
// results in a second launch, and for the dequantized weight slabs of the
// prefill routes.  The reference's entry points take no workspace argument;
// its only device allocations (the topsaten MoE workspaces) go through a
// stream-ordered allocator the host registers
// (kernels/topsaten_moe_wrapper.cpp:18-48).  Here likewise:
//  * with an allocator registered (ubridge_set_workspace_allocator), every
//    call that needs scratch takes it from that allocator on its stream and
//    hands it back on the same stream once its kernels are enqueued; the
//    library then holds no device memory of its own;
//  * otherwise a per-(device, stream) pool buffer, grown on demand.  A buffer
//    it outgrows is retired: freed once an event recorded after its last use
//    has completed, unless it was handed out while the stream captured a
//    graph (graphs keep its address: it then lives until
//    ubridge_release_workspace).  ubridge_release_workspace(stream)
//    synchronizes the stream and frees all of that stream's buffers.
// Growth during a graph capture allocates with the capture mode relaxed, so
// calls take the same route (and give the same bits) captured or eager.
#include <map>
#include <mutex>
#include <utility>
#include <vector>
namespace {
struct WsBuf {
  void* p = nullptr;
  size_t bytes = 0;
  bool graph = false;  // handed out during a capture
};
struct WsRetired {
  WsBuf b;
  hipEvent_t ev = nullptr;  // completes after the buffer's last eager use
};
struct WsPool {
  WsBuf cur;
  std::vector<WsRetired> retired;  // ev null: not yet ordered (see sweep)
};
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, WsPool> g_ws;
size_t g_ws_live_n = 0, g_ws_live_bytes = 0;  // pool buffers allocated, not freed
long g_ws_caller_out = 0;                     // caller-allocator blocks not yet handed back
ubridge_ws_alloc_fn g_ws_alloc = nullptr;
ubridge_ws_free_fn g_ws_free = nullptr;
void* g_ws_ctx = nullptr;

bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return st != hipStreamCaptureStatusNone;
}

void ws_free(const WsBuf& b) {
  if (!b.p) return;
  (void)hipFree(b.p);
  (void)hipGetLastError();
  g_ws_live_n--;
  g_ws_live_bytes -= b.bytes;
}

// Retired buffers of a pool (s not capturing, caller holds g_ws_mu): order
// the unordered ones behind an event recorded now (everything that used them
// is already on s), free those whose event has completed.  Graph-held
// buffers stay until released.
void ws_sweep(WsPool& pool, hipStream_t s) {
  for (size_t i = 0; i < pool.retired.size();) {
    WsRetired& r = pool.retired[i];
    if (r.b.graph) {
      i++;
      continue;
    }
    if (!r.ev) {
      if (hipEventCreateWithFlags(&r.ev, hipEventDisableTiming) != hipSuccess ||
          hipEventRecord(r.ev, s) != hipSuccess) {
        (void)hipGetLastError();
        if (r.ev) (void)hipEventDestroy(r.ev);
        r.ev = nullptr;
        i++;
        continue;
      }
    }
    if (hipEventQuery(r.ev) == hipSuccess) {
      (void)hipEventDestroy(r.ev);
      ws_free(r.b);
      pool.retired.erase(pool.retired.begin() + i);
    } else {
      (void)hipGetLastError();  // hipErrorNotReady
      i++;
    }
  }
}

void* ws_pool_get(hipStream_t s, size_t bytes) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  const bool cap = capturing(s);
  std::lock_guard<std::mutex> lk(g_ws_mu);
  WsPool& pool = g_ws[{dev, s}];
  if (!cap && !pool.retired.empty()) ws_sweep(pool, s);
  if (pool.cur.bytes >= bytes) {
    pool.cur.graph |= cap;
    return pool.cur.p;
  }
  void* p = nullptr;
  const size_t sz = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
  hipError_t e;
  {
    UbRelaxCapture relax;
    e = hipMalloc(&p, sz);
  }
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  g_ws_live_n++;
  g_ws_live_bytes += sz;
  if (pool.cur.p) {
    pool.retired.push_back(WsRetired{pool.cur, nullptr});
    if (!cap) ws_sweep(pool, s);  // orders it behind the work already on s
  }
  pool.cur = WsBuf{p, sz, cap};
  return p;
}
}  // namespace

UbScratch::UbScratch(hipStream_t s, size_t bytes) : s_(s) {
  if (bytes == 0) return;
  ubridge_ws_alloc_fn fa;
  void* ctx;
  {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    fa = g_ws_alloc;
    ctx = g_ws_ctx;
  }
  if (fa) {
    void* p = nullptr;
    if (fa(&p, bytes, (void*)s, ctx) == 0 && p) {
      p_ = p;
      caller_ = true;
      std::lock_guard<std::mutex> lk(g_ws_mu);
      g_ws_caller_out++;
    }
    return;
  }
  p_ = ws_pool_get(s, bytes);
}

UbScratch::~UbScratch() {
  if (!caller_) return;
  ubridge_ws_free_fn ff;
  void* ctx;
  {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    ff = g_ws_free;
    ctx = g_ws_ctx;
    g_ws_caller_out--;
  }
  if (ff) ff(p_, (void*)s_, ctx);
}

UB_API int ubridge_set_workspace_allocator(ubridge_ws_alloc_fn alloc, ubridge_ws_free_fn free_fn,
                                           void* ctx) {
  if ((alloc == nullptr) != (free_fn == nullptr))
    return ub_set_error(UB_ERR_INVALID_ARG,
                        "ubridge_set_workspace_allocator: give both functions or neither");
  std::lock_guard<std::mutex> lk(g_ws_mu);
  g_ws_alloc = alloc;
  g_ws_free = free_fn;
  g_ws_ctx = ctx;
  return UB_OK;
}

UB_API int ubridge_release_workspace(void* stream) {
  hipStream_t s = ub_stream(stream);
  {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    if (g_ws.empty()) return UB_OK;  // nothing to free (touches no device)
  }
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return ub_set_error(UB_ERR_LAUNCH, "no device");
  if (capturing(s))
    return ub_set_error(UB_ERR_INVALID_ARG,
                        "ubridge_release_workspace: the stream is capturing a graph");
  std::lock_guard<std::mutex> lk(g_ws_mu);
  auto it = g_ws.find({dev, s});
  if (it == g_ws.end()) return UB_OK;
  if (hipStreamSynchronize(s) != hipSuccess) {
    const hipError_t e = hipGetLastError();
    return ub_set_error(UB_ERR_LAUNCH, "ubridge_release_workspace: %s", hipGetErrorString(e));
  }
  for (WsRetired& r : it->second.retired) {
    if (r.ev) (void)hipEventDestroy(r.ev);
    ws_free(r.b);
  }
  ws_free(it->second.cur);
  g_ws.erase(it);
  return UB_OK;
}

UB_API int ubridge_workspace_stats(size_t* live_buffers, size_t* live_bytes,
                                   long* caller_blocks_out) {
  std::lock_guard<std::mutex> lk(g_ws_mu);
  if (live_buffers) *live_buffers = g_ws_live_n;
  if (live_bytes) *live_bytes = g_ws_live_bytes;
  if (caller_blocks_out) *caller_blocks_out = g_ws_caller_out;
  return UB_OK;
}
