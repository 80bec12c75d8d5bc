// blaslt.cpp -- plain dense GEMMs through hipBLASLt.
//
// matmul_{bf16,f16} beyond decode sizes is a library GEMM with nothing to
// fuse (no dequantization, no epilogue), so it goes to hipBLASLt; the
// library's own MFMA core stays the fallback.  Row-major C[M, N] = A[M, K] .
// B (B [K, N], or [N, K] with rhs_transpose) is computed as the column-major
// C^T = op(B) . A^T, so no operand is copied.  One handle per device and one
// plan (descriptors and the heuristic's algorithm) per shape, created on
// first use; no workspace, so a call allocates nothing after its plan
// exists.  A plan first needed while the stream captures a graph is made with
// the capture mode relaxed (outside the graph), so captured and eager calls
// take the same route -- once the per-device set-up below exists.  The cache keeps the kPlanCap most recently used
// plans: serving with many distinct token counts re-plans an evicted shape
// instead of growing without bound.
#include <hipblaslt/hipblaslt.h>

#include <atomic>
#include <map>
#include <mutex>
#include <tuple>

#include "common.h"

namespace {

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t lw = nullptr, la = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  bool ok = false;
  uint64_t used = 0;  // last-use tick, for eviction
};

constexpr size_t kPlanCap = 256;
uint64_t g_tick = 0;

void destroy_plan(Plan& p) {
  if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
  for (auto* l : {&p.lw, &p.la, &p.lc})
    if (*l) hipblasLtMatrixLayoutDestroy(*l);
  p = Plan{};
}

// dev dt batch M N K rhs_t bcast ldc c_f32
using Key = std::tuple<int, int, int, int, int, int, int, int, int, int>;

std::mutex g_mu;
std::map<int, hipblasLtHandle_t> g_handles;
std::map<Key, Plan> g_plans;

bool make_plan(hipblasLtHandle_t h, Plan& p, int dt, int batch, int M, int N, int K, int rhs_t,
               int bcast, int ldc, int c_f32) {
  const hipDataType t = dt == UB_BF16 ? HIP_R_16BF : HIP_R_16F;
  const hipDataType tc = c_f32 ? HIP_R_32F : t;
  // column-major views: W as N x K (rhs_t = 0: [K, N] row-major, ld N) or,
  // transposed, K x N (rhs_t = 1: [N, K] row-major, ld K); A^T K x M; C^T N x M
  if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
    return false;
  const int32_t opw = rhs_t ? HIPBLAS_OP_T : HIPBLAS_OP_N, opa = HIPBLAS_OP_N;
  if (hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opw, sizeof(opw)) ||
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opa, sizeof(opa)))
    return false;
  if (hipblasLtMatrixLayoutCreate(&p.lw, t, rhs_t ? K : N, rhs_t ? N : K, rhs_t ? K : N) ||
      hipblasLtMatrixLayoutCreate(&p.la, t, K, M, K) ||
      hipblasLtMatrixLayoutCreate(&p.lc, tc, N, M, ldc))
    return false;
  if (batch > 1) {
    const int32_t bc = batch;
    const int64_t sw = bcast ? 0 : (int64_t)K * N, sa = (int64_t)M * K, sc = (int64_t)M * ldc;
    for (auto* l : {&p.lw, &p.la, &p.lc})
      if (hipblasLtMatrixLayoutSetAttribute(*l, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &bc,
                                            sizeof(bc)))
        return false;
    if (hipblasLtMatrixLayoutSetAttribute(p.lw, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &sw,
                                          sizeof(sw)) ||
        hipblasLtMatrixLayoutSetAttribute(p.la, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &sa,
                                          sizeof(sa)) ||
        hipblasLtMatrixLayoutSetAttribute(p.lc, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &sc,
                                          sizeof(sc)))
      return false;
  }
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref)) return false;
  const uint64_t ws = 0;
  hipblasLtMatmulHeuristicResult_t res{};
  int n = 0;
  const bool got =
      hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                            sizeof(ws)) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.lw, p.la, p.lc, p.lc, pref, 1, &res, &n) ==
          HIPBLAS_STATUS_SUCCESS &&
      n > 0 && res.state == HIPBLAS_STATUS_SUCCESS && res.workspaceSize == 0;
  hipblasLtMatmulPreferenceDestroy(pref);
  if (!got) return false;
  p.algo = res.algo;
  return true;
}

// The fp8 W8A8 GEMM (ubridge_fp8_gemm's contract): out[M, N] bf16 =
// (a[M, K] . w_nk[N, K]^T) * sa[M] * sw[N], e4m3 (OCP) operands, f32
// accumulation.  Column-major: D^T N x M = op(W) . A^T with W K x N
// transposed; the row scales of the library's A operand are sw (N of
// them), of its B operand sa (M), applied as outer vectors.  The scale
// pointers are part of the plan's descriptor and are set again by each call
// (under g_mu).
bool make_plan_fp8(hipblasLtHandle_t h, Plan& p, int M, int N, int K, const float* sa,
                   const float* sw) {
  if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
    return false;
  const int32_t opw = HIPBLAS_OP_T, opa = HIPBLAS_OP_N;
  const int32_t vec = HIPBLASLT_MATMUL_MATRIX_SCALE_OUTER_VEC_32F;
  const void* pw = sw;
  const void* pa = sa;
  if (hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opw, sizeof(opw)) ||
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opa, sizeof(opa)) ||
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_A_SCALE_MODE, &vec, sizeof(vec)) ||
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_B_SCALE_MODE, &vec, sizeof(vec)) ||
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_A_SCALE_POINTER, &pw, sizeof(pw)) ||
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_B_SCALE_POINTER, &pa, sizeof(pa)))
    return false;
  if (hipblasLtMatrixLayoutCreate(&p.lw, HIP_R_8F_E4M3, K, N, K) ||
      hipblasLtMatrixLayoutCreate(&p.la, HIP_R_8F_E4M3, K, M, K) ||
      hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_16BF, N, M, N))
    return false;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref)) return false;
  const uint64_t ws = 0;
  hipblasLtMatmulHeuristicResult_t res{};
  int n = 0;
  const bool got =
      hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                            sizeof(ws)) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.lw, p.la, p.lc, p.lc, pref, 1, &res, &n) ==
          HIPBLAS_STATUS_SUCCESS &&
      n > 0 && res.state == HIPBLAS_STATUS_SUCCESS && res.workspaceSize == 0;
  hipblasLtMatmulPreferenceDestroy(pref);
  if (!got) return false;
  p.algo = res.algo;
  return true;
}
constexpr int kFp8Key = 8;  // plan-key data type of the fp8 GEMM

// hipBLASLt's per-device set-up: the handle, and one heuristic query of a
// small shape, which loads the library's kernel catalogue.  Measured on
// MI355X: made while a stream captures a graph (even with the capture mode
// relaxed), this first-time set-up ends the process; plans of new shapes
// made inside a capture once it exists are fine.  So it is made only outside
// captures: at the first call on the device of any entry point that can
// route to hipBLASLt, or by ubridge_init.  Caller holds g_mu.
std::atomic<uint64_t> g_ready{0};  // bit dev: set-up done (handle may be null)

hipblasLtHandle_t setup_locked(int dev, hipStream_t s) {
  auto hi = g_handles.find(dev);
  if (hi != g_handles.end()) return hi->second;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (cs != hipStreamCaptureStatusNone) return nullptr;
  hipblasLtHandle_t h = nullptr;
  if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) h = nullptr;
  if (h) {
    Plan warm;
    (void)make_plan(h, warm, UB_BF16, 1, 256, 256, 256, 1, 0, 256, 0);
    destroy_plan(warm);
  }
  g_handles.emplace(dev, h);
  if (dev >= 0 && dev < 64) g_ready.fetch_or(1ull << dev, std::memory_order_release);
  return h;
}

// The plan of a shape, made on first use; null when hipBLASLt cannot serve
// it, or its per-device set-up has not been made and s is capturing.
// Caller holds g_mu.
const Plan* plan_of(int dt, int batch, int M, int N, int K, int rhs_t, int bcast, int ldc, int c_f32,
                    hipStream_t s, int& dev, const float* sa = nullptr, const float* sw = nullptr) {
  if ((dt != UB_BF16 && dt != UB_F16 && dt != kFp8Key) || batch < 1 || M < 1 || N < 1 || K < 1 ||
      ldc < N)
    return nullptr;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  const Key key{dev, dt, batch, M, N, K, rhs_t, bcast, ldc, c_f32};
  auto it = g_plans.find(key);
  if (it == g_plans.end()) {
    hipblasLtHandle_t h = setup_locked(dev, s);
    if (!h) return nullptr;
    UbRelaxCapture relax;  // legal (and outside the graph) if s is capturing
    if (g_plans.size() >= kPlanCap) {  // evict the least recently used
      auto lru = g_plans.begin();
      for (auto j = g_plans.begin(); j != g_plans.end(); ++j)
        if (j->second.used < lru->second.used) lru = j;
      destroy_plan(lru->second);
      g_plans.erase(lru);
    }
    Plan p;
    p.ok = dt == kFp8Key ? make_plan_fp8(h, p, M, N, K, sa, sw)
                         : make_plan(h, p, dt, batch, M, N, K, rhs_t, bcast, ldc, c_f32);
    it = g_plans.emplace(key, p).first;
  }
  it->second.used = ++g_tick;
  return it->second.ok ? &it->second : nullptr;
}

}  // namespace

// Per-device hipBLASLt set-up at the first call that can route to it (see
// setup_locked); a no-op once made, and while s is capturing.
void ub_blaslt_prepare(hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return;
  }
  if (dev >= 0 && dev < 64 && (g_ready.load(std::memory_order_acquire) >> dev & 1)) return;
  std::lock_guard<std::mutex> lk(g_mu);
  (void)setup_locked(dev, s);
}

// ubridge_init: the per-device set-up of the current device, now.  For a
// process whose first library call would be made inside a graph capture.
UB_API int ubridge_init(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    const hipError_t e = hipGetLastError();
    return ub_set_error(UB_ERR_LAUNCH, "ubridge_init: %s", hipGetErrorString(e));
  }
  std::lock_guard<std::mutex> lk(g_mu);
  if (!setup_locked(dev, nullptr))
    return ub_set_error(UB_ERR_LAUNCH, "ubridge_init: hipBLASLt set-up failed");
  return UB_OK;
}

// Whether ub_blaslt_gemm can serve this shape (making its plan now).
bool ub_blaslt_ready(int batch, int M, int N, int K, int rhs_t, int bcast, int ldc, int c_f32,
                     int dt, hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_mu);
  int dev = 0;
  return plan_of(dt, batch, M, N, K, rhs_t, bcast, ldc, c_f32, s, dev) != nullptr;
}

// C = A . B through hipBLASLt (see above), C with leading dimension ldc (in
// elements; f32 when c_f32, else the input type); UB_ERR_UNSUPPORTED when it
// cannot serve the call (nothing recorded: the caller falls back).
int ub_blaslt_gemm(const void* a, const void* b, void* c, int batch, int M, int N, int K,
                   int rhs_t, int bcast, int ldc, int c_f32, int dt, hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_mu);
  int dev = 0;
  const Plan* p = plan_of(dt, batch, M, N, K, rhs_t, bcast, ldc, c_f32, s, dev);
  if (!p) return UB_ERR_UNSUPPORTED;
  const float alpha = 1.f, beta = 0.f;
  if (hipblasLtMatmul(g_handles[dev], p->desc, &alpha, b, p->lw, a, p->la, &beta, c, p->lc, c,
                      p->lc, &p->algo, nullptr, 0, s) != HIPBLAS_STATUS_SUCCESS)
    return ub_set_error(UB_ERR_LAUNCH, "hipblasLtMatmul failed");
  return UB_OK;
}

// The fp8 W8A8 GEMM through hipBLASLt (make_plan_fp8); UB_ERR_UNSUPPORTED
// when it cannot serve the shape (nothing recorded: the caller falls back).
int ub_blaslt_fp8(const uint8_t* a, const float* sa, const uint8_t* w_nk, const float* sw,
                  void* out, int M, int K, int N, hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_mu);
  int dev = 0;
  const Plan* p = plan_of(kFp8Key, 1, M, N, K, 1, 0, N, 0, s, dev, sa, sw);
  if (!p) return UB_ERR_UNSUPPORTED;
  const void* pw = sw;
  const void* pa = sa;
  if (hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_A_SCALE_POINTER, &pw,
                                      sizeof(pw)) ||
      hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_B_SCALE_POINTER, &pa,
                                      sizeof(pa)))
    return ub_set_error(UB_ERR_LAUNCH, "hipBLASLt fp8 scale pointers");
  const float alpha = 1.f, beta = 0.f;
  if (hipblasLtMatmul(g_handles[dev], p->desc, &alpha, w_nk, p->lw, a, p->la, &beta, out, p->lc,
                      out, p->lc, &p->algo, nullptr, 0, s) != HIPBLAS_STATUS_SUCCESS)
    return ub_set_error(UB_ERR_LAUNCH, "hipblasLtMatmul (fp8) failed");
  return UB_OK;
}
