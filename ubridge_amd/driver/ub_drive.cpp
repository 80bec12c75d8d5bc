// ub_drive.cpp -- C++ host driver over the C ABI of libubridge_hip.so.
//
// Issues the reference's hot-path call sequences the way its Rust host
// (candle-gcu over src/ffi.rs and the name-keyed launch of
// src/gcu_device.rs:160-198 / src/gcu_launch.rs:121-193) issues them, next
// to the fused forms this library adds, checks that each pair agrees and
// times both with HIP events:
//
//   qmatmul   GGUF QMatMul, Q4_K: dequantize_block_q4_k_bf16 ("quant") then
//             get_gemm_launch_params + matmul_bf16 ("matmul"), both launched
//             by name, against ubridge_qmatmul (one fused GEMV).
//   w4a16     get_gemm_launch_params + matmul_bf16_4bit by name, against the
//             host-lib dequant_bf16 + matmul_bf16 (dense weight in HBM).
//   moe       topk_softmax_f32 -> moe_align_block_size -> invoke_fused_moe
//             (gate/up) -> silu_and_mul -> invoke_fused_moe (down, routed
//             weight) -> k-slot sum; the status-returning topsaten_* names
//             on the same inputs must reproduce its routing and gate/up rows.
//   workspace ubridge_w4a16_gemm on a K-split shape (scratch partials) with
//             the library's stream pool, then with a caller allocator
//             (hipMallocAsync / hipFreeAsync) registered through
//             ubridge_set_workspace_allocator, eagerly and captured into a
//             HIP graph replayed twice: all outputs bit-identical, no caller
//             block outstanding, the pool freed before the stream is.
//
// Only the C ABI is used for compute; HIP is used for memory, the stream and
// events.  One JSON line per sequence on stdout; exit status 0 when every
// check passes.
//
//   ub_drive [--quick] [--reps R]
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "ubridge_hip.h"

namespace {

constexpr int kBf16 = 2;                         // library dtype code
constexpr int kQ4K = 12;                         // GGML id of Q4_K
constexpr int kDataBf16 = 5, kDataI4 = 15;       // reference DATATYPE codes (src/lib.rs:88-106)

int g_fail = 0;

#define HIP_OK(x)                                                                       \
  do {                                                                                  \
    hipError_t e_ = (x);                                                                \
    if (e_ != hipSuccess) {                                                             \
      std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      std::exit(2);                                                                     \
    }                                                                                   \
  } while (0)

void lib_ok(int rc, const char* what) {
  const int e = rc ? rc : ubridge_last_error();
  if (e) {
    std::fprintf(stderr, "%s: error %d: %s\n", what, e, ubridge_last_error_string());
    std::exit(3);
  }
}

// f32 -> bf16 bits, round to nearest even (finite inputs)
uint16_t to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
float from_bf16(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

template <class T>
struct Buf {  // device buffer with a host mirror
  std::vector<T> h;
  T* d = nullptr;
  explicit Buf(size_t n) : h(n) { HIP_OK(hipMalloc(&d, n * sizeof(T) + 16)); }
  ~Buf() { (void)hipFree(d); }
  Buf(const Buf&) = delete;
  Buf& operator=(const Buf&) = delete;
  void up() { HIP_OK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice)); }
  void down() { HIP_OK(hipMemcpy(h.data(), d, h.size() * sizeof(T), hipMemcpyDeviceToHost)); }
};

double rel_err_bf16(const std::vector<uint16_t>& got, const std::vector<uint16_t>& want) {
  double num = 0, den = 0;
  for (size_t i = 0; i < got.size(); i++) {
    const double g = from_bf16(got[i]), w = from_bf16(want[i]);
    if (!std::isfinite(g)) return INFINITY;
    num += (g - w) * (g - w);
    den += w * w;
  }
  return std::sqrt(num / (den > 0 ? den : 1));
}

// microseconds per call of fn, over reps back-to-back calls on s
template <class F>
double time_us(hipStream_t s, int reps, F fn) {
  fn();
  HIP_OK(hipStreamSynchronize(s));
  hipEvent_t a, b;
  HIP_OK(hipEventCreate(&a));
  HIP_OK(hipEventCreate(&b));
  HIP_OK(hipEventRecord(a, s));
  for (int i = 0; i < reps; i++) fn();
  HIP_OK(hipEventRecord(b, s));
  HIP_OK(hipEventSynchronize(b));
  float ms = 0;
  HIP_OK(hipEventElapsedTime(&ms, a, b));
  HIP_OK(hipEventDestroy(a));
  HIP_OK(hipEventDestroy(b));
  return 1e3 * ms / reps;
}

void check(bool ok, const char* what) {
  if (!ok) {
    std::fprintf(stderr, "check failed: %s\n", what);
    g_fail++;
  }
}

// Name-keyed launch, as GcuLaunchAsync::launch passes its parameter tuple.
void launch(const char* name, const char* module, std::vector<void*> args, hipStream_t s) {
  const void* f = ubridge_get_function(name, module);
  if (!f) {
    std::fprintf(stderr, "no kernel %s in module %s\n", name, module);
    std::exit(3);
  }
  lib_ok(ubridge_launch(f, args.data(), s), name);
}

// The 17 shared matmul arguments from the launch parameters, in order.
struct MmArgs {
  int dtype, batch, m, k, n, lhs_mc, rhs_mc, batch_mc, lhs_t, rhs_t;
  float alpha, beta, addmm_beta;
  int sip_m, sip_k, sip_n, bcast;
  void push(std::vector<void*>& v) {
    for (void* p : {(void*)&dtype, (void*)&batch, (void*)&m, (void*)&k, (void*)&n, (void*)&lhs_mc,
                    (void*)&rhs_mc, (void*)&batch_mc, (void*)&lhs_t, (void*)&rhs_t, (void*)&alpha,
                    (void*)&beta, (void*)&addmm_beta, (void*)&sip_m, (void*)&sip_k, (void*)&sip_n,
                    (void*)&bcast})
      v.push_back(p);
  }
};
MmArgs mm_args(int wtype, int m, int k, int n, int rhs_t) {
  const UbridgeGemmOpParas* p = ubridge_get_gemm_launch_params(kDataBf16, wtype, 1, m, k, n, rhs_t);
  if (!p) lib_ok(ubridge_last_error(), "get_gemm_launch_params");
  return MmArgs{kBf16, 1, m, k, n, p->lhs_multicore, p->rhs_multicore, p->batch_multicore, 0,
                rhs_t, 1.f, 0.f, 0.f, p->sip_m, p->sip_k, p->sip_n, 1};
}

// ---------------------------------------------------------------- (B)
void run_qmatmul(hipStream_t s, int M, int K, int N, int reps, std::mt19937& rng) {
  const size_t nb = (size_t)N * K / 256;
  Buf<int8_t> w(nb * 144);  // SoA Q4_K: nb x 16-byte headers, then nb x 128 code bytes
  std::uniform_int_distribution<int> byte(0, 255), dpick(0, 3);
  const uint16_t dvals[4] = {0x1c00, 0x1e00, 0x2000, 0x2100};  // f16 2^-8 .. 2^-7 * 1.25
  for (size_t b = 0; b < nb; b++) {
    uint8_t* h = (uint8_t*)&w.h[b * 16];
    const uint16_t d = dvals[dpick(rng)], dm = dvals[dpick(rng)];
    std::memcpy(h, &d, 2);
    std::memcpy(h + 2, &dm, 2);
    for (int i = 4; i < 16; i++) h[i] = (uint8_t)byte(rng);
  }
  for (size_t i = nb * 16; i < nb * 144; i++) w.h[i] = (int8_t)byte(rng);
  Buf<uint16_t> x((size_t)M * K), wd((size_t)N * K), y_ref((size_t)M * N), y((size_t)M * N);
  std::normal_distribution<float> nd(0.f, 1.f);
  for (auto& v : x.h) v = to_bf16(nd(rng));
  w.up();
  x.up();
  const size_t ws_bytes = ubridge_qmatmul_workspace_size(kQ4K, M, K);
  void* ws = nullptr;
  HIP_OK(hipMalloc(&ws, ws_bytes + 16));

  size_t numel = (size_t)N * K;
  MmArgs mm = mm_args(kDataBf16, M, K, N, 1);  // y = x . Wd^T, Wd [N, K]
  auto reference = [&]() {
    launch("dequantize_block_q4_k_bf16", "quant", {&w.d, &wd.d, &numel}, s);
    std::vector<void*> a = {&x.d, &wd.d, &y_ref.d};
    mm.push(a);
    launch("matmul_bf16", "matmul", a, s);
  };
  auto fused = [&]() {
    lib_ok(ubridge_qmatmul(kQ4K, w.d, x.d, kBf16, y.d, kBf16, M, N, K, ws, ws_bytes, s),
           "ubridge_qmatmul");
  };
  const double t_ref = time_us(s, reps, reference), t_fused = time_us(s, reps, fused);
  y_ref.down();
  y.down();
  // the fused GEMV quantizes activations to Q8_K (Candle's method), the
  // reference path rounds the weight to bf16: a few 1e-3 apart, up to ~2e-2
  // where random sub-block mins cancel most of an output
  const double e = rel_err_bf16(y.h, y_ref.h);
  check(e < 3e-2, "qmatmul: fused vs dequantize + matmul_bf16");
  const double wbytes = (double)nb * 144;
  std::printf("{\"sequence\": \"qmatmul\", \"qtype\": \"q4_k\", \"M\": %d, \"K\": %d, \"N\": %d, "
              "\"reference_us\": %.2f, \"fused_us\": %.2f, \"fused_weight_GBps\": %.1f, "
              "\"rel_err\": %.3e}\n",
              M, K, N, t_ref, t_fused, wbytes / t_fused / 1e3, e);
  (void)hipFree(ws);
}

// ---------------------------------------------------------------- (C)
void run_w4a16(hipStream_t s, int M, int K, int N, int G, int reps, std::mt19937& rng) {
  Buf<uint8_t> q((size_t)K / 2 * N);
  Buf<uint16_t> a((size_t)M * K), sc((size_t)K / G * N), zr((size_t)K / G * N);
  Buf<uint16_t> wd((size_t)K * N), y_ref((size_t)M * N), y((size_t)M * N);
  std::uniform_int_distribution<int> byte(0, 255), z16(0, 15);
  std::uniform_real_distribution<float> su(0.002f, 0.02f);
  std::normal_distribution<float> nd(0.f, 1.f);
  for (auto& v : q.h) v = (uint8_t)byte(rng);
  for (auto& v : a.h) v = to_bf16(nd(rng));
  for (auto& v : sc.h) v = to_bf16(su(rng));
  for (auto& v : zr.h) v = to_bf16((float)z16(rng));
  q.up();
  a.up();
  sc.up();
  zr.up();
  MmArgs m4 = mm_args(kDataI4, M, K, N, 0);
  int group = G;
  auto by_name = [&]() {
    std::vector<void*> v = {&a.d, &q.d, &y.d, &sc.d, &zr.d};
    m4.push(v);
    v.push_back(&group);
    launch("matmul_bf16_4bit", "matmul", v, s);
  };
  MmArgs md = mm_args(kDataBf16, M, K, N, 0);
  auto dense = [&]() {
    dequant_bf16(wd.d, q.d, sc.d, zr.d, K / 2, N, 0, G, s);
    lib_ok(0, "dequant_bf16");
    std::vector<void*> v = {&a.d, &wd.d, &y_ref.d};
    md.push(v);
    launch("matmul_bf16", "matmul", v, s);
  };
  const double t4 = time_us(s, reps, by_name), td = time_us(s, reps, dense);
  y.down();
  y_ref.down();
  const double e = rel_err_bf16(y.h, y_ref.h);
  check(e < 1e-2, "w4a16: matmul_bf16_4bit vs dequant_bf16 + matmul_bf16");
  std::printf("{\"sequence\": \"w4a16\", \"M\": %d, \"K\": %d, \"N\": %d, \"group\": %d, "
              "\"sip_m\": %d, \"sip_n\": %d, \"matmul_bf16_4bit_us\": %.2f, "
              "\"dequant_then_dense_us\": %.2f, \"TFLOPs\": %.1f, \"rel_err\": %.3e}\n",
              M, K, N, G, m4.sip_m, m4.sip_n, t4, td, 2.0 * M * K * N / t4 / 1e6, e);
}

// ---------------------------------------------------------------- (D)
void run_moe(hipStream_t s, int T, int E, int k, int H, int I, int bs, int reps,
             std::mt19937& rng) {
  const int slots = T * k, max_pad = slots + E * (bs - 1), max_blk = max_pad / bs;
  Buf<float> logits((size_t)T * E), tw((size_t)slots), tw2((size_t)slots);
  Buf<int> ids(slots), ids2(slots), tei(slots), sorted(max_pad), sorted2(max_pad), eids(max_blk),
      eids2(max_blk), ntpp(1), ntpp2(1);
  Buf<uint16_t> x((size_t)T * H), w13((size_t)E * 2 * I * H), w2((size_t)E * H * I);
  Buf<uint16_t> c1((size_t)slots * 2 * I), c1b((size_t)slots * 2 * I), act((size_t)slots * I),
      c2((size_t)slots * H), y((size_t)T * H);
  std::normal_distribution<float> nd(0.f, 1.f);
  for (auto& v : logits.h) v = nd(rng);
  for (auto& v : x.h) v = to_bf16(nd(rng));
  for (auto& v : w13.h) v = to_bf16(0.05f * nd(rng));
  for (auto& v : w2.h) v = to_bf16(0.05f * nd(rng));
  logits.up();
  x.up();
  w13.up();
  w2.up();
  auto chain = [&]() {
    topk_softmax_f32(logits.d, tw.d, ids.d, T, E, k, 1, s);
    moe_align_block_size(sorted.d, eids.d, ntpp.d, ids.d, nullptr, nullptr, E, bs, T, k, s);
    invoke_fused_moe_bf16(c1.d, x.d, w13.d, nullptr, tw.d, sorted.d, eids.d, ntpp.d, T, H, 2 * I,
                          E, slots, k, bs, 0, 0, s);
    lib_ok(ubridge_silu_and_mul(act.d, c1.d, slots, I, kBf16, s), "silu_and_mul");
    invoke_fused_moe_bf16(c2.d, act.d, w2.d, nullptr, tw.d, sorted.d, eids.d, ntpp.d, slots, I, H,
                          E, slots, k, bs, 1, 0, s);
    lib_ok(ubridge_moe_sum(y.d, c2.d, T, k, H, kBf16, s), "moe_sum");
  };
  const double t_chain = time_us(s, reps, chain);
  lib_ok(ubridge_device_error(s), "moe chain device flag");
  // the status-returning names on the same inputs
  lib_ok(topsaten_topk_softmax_f32(logits.d, tw2.d, ids2.d, tei.d, T, E, k, 1, s), "topsaten topk");
  lib_ok(topsaten_moe_align_block_size(sorted2.d, eids2.d, ntpp2.d, ids2.d, T, k, E, bs, s),
         "topsaten align");
  lib_ok(topsaten_fused_moe_gemm(c1b.d, x.d, w13.d, tw2.d, ids2.d, sorted2.d, eids2.d, ntpp2.d, 0,
                                 k, bs, T, H, 2 * I, E, 5 /* bf16 */, s),
         "topsaten fused_moe_gemm");
  HIP_OK(hipStreamSynchronize(s));
  for (auto* b : {&ids, &ids2, &tei, &sorted, &sorted2, &eids, &eids2, &ntpp, &ntpp2}) b->down();
  tw.down();
  tw2.down();
  c1.down();
  c1b.down();
  y.down();
  check(ids.h == ids2.h && std::memcmp(tw.h.data(), tw2.h.data(), slots * 4) == 0,
        "moe: topsaten_topk_softmax_f32 == topk_softmax_f32");
  bool tei_ok = true;
  for (int t = 0; t < T; t++)
    for (int j = 0; j < k; j++) tei_ok &= tei.h[t * k + j] == j * T + t;
  check(tei_ok, "moe: token_expert_indices");
  check(sorted.h == sorted2.h && eids.h == eids2.h && ntpp.h == ntpp2.h,
        "moe: topsaten_moe_align_block_size == moe_align_block_size");
  // align invariants: padded total, every slot exactly once, one expert per block
  const int npad = ntpp.h[0];
  std::vector<int> seen(slots, 0);
  bool inv = npad % bs == 0 && npad <= max_pad;
  for (int i = 0; i < npad && inv; i++) {
    const int v = sorted.h[i];
    if (v < slots) {
      seen[v]++;
      inv &= ids.h[v] == eids.h[i / bs];
    } else {
      inv &= v == slots;
    }
  }
  for (int v : seen) inv &= v == 1;
  check(inv, "moe: align invariants");
  // both gate/up GEMM forms on the same routing: identical rows for real slots
  bool same = true;
  for (int i = 0; i < npad; i++) {
    const int v = sorted.h[i];
    if (v < slots)
      same &= std::memcmp(&c1.h[(size_t)v * 2 * I], &c1b.h[(size_t)v * 2 * I], 2 * I * 2) == 0;
  }
  check(same, "moe: topsaten_fused_moe_gemm == invoke_fused_moe_bf16 (gate/up)");
  bool finite = true;
  for (uint16_t v : y.h) finite &= std::isfinite(from_bf16(v));
  check(finite, "moe: finite output");
  std::printf("{\"sequence\": \"moe\", \"T\": %d, \"E\": %d, \"top_k\": %d, \"H\": %d, \"I\": %d, "
              "\"block_size\": %d, \"chain_us\": %.2f, \"num_tokens_post_pad\": %d}\n",
              T, E, k, H, I, bs, t_chain, npad);
}

// ---------------------------------------------------------------- (E)
struct AsyncAlloc {  // stream-ordered caller allocator over hipMallocAsync
  long calls = 0, live = 0;
  static int alloc(void** p, size_t bytes, void* stream, void* ctx) {
    auto* a = static_cast<AsyncAlloc*>(ctx);
    if (hipMallocAsync(p, bytes, (hipStream_t)stream) != hipSuccess) return 1;
    a->calls++;
    a->live++;
    return 0;
  }
  static void release(void* p, void* stream, void* ctx) {
    auto* a = static_cast<AsyncAlloc*>(ctx);
    (void)hipFreeAsync(p, (hipStream_t)stream);
    a->live--;
  }
};

void run_workspace(hipStream_t s, int M, int K, int N, int G, std::mt19937& rng) {
  Buf<int32_t> qw((size_t)K / 8 * N), qz((size_t)K / G * N / 8);
  Buf<uint16_t> a((size_t)M * K), sc((size_t)K / G * N);
  Buf<uint16_t> y_pool((size_t)M * N), y_cb((size_t)M * N), y_graph((size_t)M * N);
  std::uniform_int_distribution<uint32_t> word;
  std::uniform_real_distribution<float> su(0.002f, 0.02f);
  std::normal_distribution<float> nd(0.f, 1.f);
  for (auto& v : qw.h) v = (int32_t)word(rng);
  for (auto& v : qz.h) v = (int32_t)word(rng);
  for (auto& v : a.h) v = to_bf16(nd(rng));
  for (auto& v : sc.h) v = to_bf16(su(rng));
  qw.up();
  qz.up();
  a.up();
  sc.up();
  auto gemm = [&](uint16_t* y) {
    lib_ok(ubridge_w4a16_gemm(a.d, qw.d, sc.d, qz.d, y, M, K, N, G, kBf16, s), "w4a16_gemm");
  };
  size_t n0 = 0, b0 = 0, n1 = 0, b1 = 0;
  long out = 0;
  lib_ok(ubridge_release_workspace(s), "release_workspace");  // earlier sequences' buffer
  lib_ok(ubridge_workspace_stats(&n0, &b0, &out), "workspace_stats");
  gemm(y_pool.d);  // library pool
  HIP_OK(hipStreamSynchronize(s));
  lib_ok(ubridge_workspace_stats(&n1, &b1, &out), "workspace_stats");
  const bool pool_used = n1 == n0 + 1 && b1 > b0;
  AsyncAlloc al;
  lib_ok(ubridge_set_workspace_allocator(&AsyncAlloc::alloc, &AsyncAlloc::release, &al),
         "set_workspace_allocator");
  gemm(y_cb.d);  // eager, caller allocator
  HIP_OK(hipStreamSynchronize(s));
  const long eager_calls = al.calls;
  hipGraph_t g;
  hipGraphExec_t ge;
  HIP_OK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
  gemm(y_graph.d);  // captured: the allocation and free become graph nodes
  HIP_OK(hipStreamEndCapture(s, &g));
  HIP_OK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
  bool graph_same = true;
  for (int r = 0; r < 2; r++) {
    HIP_OK(hipMemsetAsync(y_graph.d, 0, y_graph.h.size() * 2, s));
    HIP_OK(hipGraphLaunch(ge, s));
    HIP_OK(hipStreamSynchronize(s));
    y_graph.down();
    y_pool.down();
    graph_same &= y_graph.h == y_pool.h;
  }
  HIP_OK(hipGraphExecDestroy(ge));
  HIP_OK(hipGraphDestroy(g));
  lib_ok(ubridge_set_workspace_allocator(nullptr, nullptr, nullptr), "set_workspace_allocator");
  size_t n2 = 0, b2 = 0;
  lib_ok(ubridge_workspace_stats(&n2, &b2, &out), "workspace_stats");
  y_cb.down();
  check(y_cb.h == y_pool.h, "workspace: caller allocator == library pool (eager)");
  check(graph_same, "workspace: captured caller-allocator replays == library pool");
  check(eager_calls >= 1 && al.calls > eager_calls && al.live == 0 && out == 0,
        "workspace: every caller block handed back");
  check(n2 == n1 && b2 == b1, "workspace: pool did not grow under the caller allocator");
  lib_ok(ubridge_release_workspace(s), "release_workspace");
  size_t n3 = 0, b3 = 0;
  lib_ok(ubridge_workspace_stats(&n3, &b3, &out), "workspace_stats");
  check(pool_used && n3 == n0, "workspace: release frees the stream's pool buffer");
  std::printf("{\"sequence\": \"workspace\", \"M\": %d, \"K\": %d, \"N\": %d, "
              "\"pool_bytes\": %zu, \"caller_allocs\": %ld, \"pool_buffers_after_release\": %zu}\n",
              M, K, N, b1 - b0, al.calls, n3);
}

}  // namespace

int main(int argc, char** argv) {
  bool quick = false;
  int reps = 20;
  for (int i = 1; i < argc; i++) {
    if (!std::strcmp(argv[i], "--quick")) quick = true;
    else if (!std::strcmp(argv[i], "--reps") && i + 1 < argc) reps = std::atoi(argv[++i]);
    else {
      std::fprintf(stderr, "usage: %s [--quick] [--reps R]\n", argv[0]);
      return 1;
    }
  }
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) {
    std::fprintf(stderr, "no GPU\n");
    return 2;
  }
  hipStream_t s;
  HIP_OK(hipStreamCreate(&s));
  std::mt19937 rng(0x5EED);
  if (quick) {
    run_qmatmul(s, 1, 1024, 512, reps, rng);
    run_qmatmul(s, 64, 1024, 512, reps, rng);  // the prefill GEMM (K split over workgroups)
    run_w4a16(s, 40, 1024, 384, 128, reps, rng);
    run_w4a16(s, 64, 512, 384, 128, reps, rng);
    run_moe(s, 40, 16, 4, 256, 128, 16, reps, rng);
  } else {
    run_qmatmul(s, 1, 4096, 14336, reps, rng);
    run_qmatmul(s, 512, 4096, 14336, reps, rng);
    run_w4a16(s, 16, 4096, 14336, 128, reps, rng);
    run_w4a16(s, 64, 4096, 14336, 128, reps, rng);
    run_moe(s, 256, 128, 8, 2048, 768, 32, reps, rng);
  }
  run_workspace(s, 72, 4096, 1544, 128, rng);  // 8 tiles: K split over workgroups
  lib_ok(ubridge_release_workspace(s), "release_workspace");
  HIP_OK(hipStreamDestroy(s));
  std::printf("{\"checks_failed\": %d}\n", g_fail);
  return g_fail ? 1 : 0;
}
