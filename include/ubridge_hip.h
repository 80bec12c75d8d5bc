/*
 * ubridge_hip.h -- C ABI of libubridge_hip.so, the MI355X (gfx950) drop-in
 * for Ubridge's quantized-matmul path.
 *
 * Conventions shared by every entry point:
 *   - All pointers are device pointers the caller allocated.  Some routes
 *     need device scratch beyond the inputs and outputs: the f32 partials of
 *     the narrow decode GEMV (matmul_* / ubridge_w4a16_gemm at <= 16 tokens,
 *     N < 8192: at most 8 x 16 x N x 4 bytes), the dequantized weight slab
 *     (at most 256 MB) of ubridge_qmatmul at prefill sizes and of the
 *     quantized matmul_* / ubridge_w4a16_gemm beyond 1024 tokens (uint8
 *     4-bit: from 640), and the f32 partials (at most 8 x M x N x 4 bytes)
 *     of the pipelined GEMMs when they split K over workgroups.  That
 *     scratch comes from the allocator the caller registers with
 *     ubridge_set_workspace_allocator (taken and handed back on the call's
 *     stream, as the reference's topsaten workspaces are), else from a
 *     per-(device, stream) library pool that ubridge_release_workspace
 *     frees.  The route a call takes depends on its shape and the tuning
 *     knobs only -- not on whether the stream is capturing a graph or an
 *     eager call came first -- so captured and eager calls give the same
 *     bits.  hipBLASLt's handle and per-shape plans (dense matmul_* above
 *     16 tokens and the slab GEMMs) are objects the library keeps; the
 *     handle is made at the first call on a device of matmul_*,
 *     ubridge_w4a16_gemm or ubridge_qmatmul made outside a capture (or by
 *     ubridge_init), since making it inside a capture is not possible: in a
 *     process whose first such call is captured, call ubridge_init first,
 *     or those captured calls take the in-house GEMMs instead of hipBLASLt.
 *   - `stream` is a hipStream_t (NULL = default stream); every call is
 *     asynchronous on it and ordered with the caller's other work.
 *   - bf16 / f16 tensors are passed as 16-bit storage (void* / uint16_t*).
 *   - Entry points that keep the reference's `void` signature record failures
 *     in a sticky per-thread error read (and cleared) by ubridge_last_error();
 *     entry points new to this library return that code directly (0 = OK).
 *   - Reference citations are EnflameTechnology/Ubridge paths.
 */
#ifndef UBRIDGE_HIP_H
#define UBRIDGE_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- errors */
/* Replaces the device-side op_assert trap (kernels/utils/moe_kernel_compat.h:
 * 115-123) and the println-only launch failure (src/gcu_launch.rs:321-323). */
int ubridge_last_error(void);               /* 0 ok, 1 arg, 2 launch, 3 unsupported, 4 index */
const char* ubridge_last_error_string(void);
const char* ubridge_version(void);

/* ------------------------------------------------------- device scratch
 * No counterpart in the reference's ffi.rs table: its kernels take no
 * workspace, and its one allocating component (topsaten) draws on a
 * stream-ordered allocator the host registers
 * (kernels/topsaten_moe_wrapper.cpp:18-48, topsatenMallocAsyncFuncRegister).
 *
 * ubridge_set_workspace_allocator: from then on every call that needs
 * scratch calls alloc(&ptr, bytes, stream, ctx) (0 = success) before its
 * launches and free_fn(ptr, stream, ctx) on the same stream right after
 * enqueueing them; the allocator must be stream-ordered (memory handed back
 * on a stream may be reused only by work ordered after it on that stream,
 * e.g. hipMallocAsync / hipFreeAsync, or torch's caching allocator) and, if
 * calls are captured into graphs, capture-aware.  Both NULL restores the
 * library pool.  Returns 1 if exactly one of the two is NULL.
 *
 * ubridge_release_workspace: synchronizes `stream` and frees every pool
 * buffer of (current device, stream), including buffers graphs captured on
 * it still name (do not replay those graphs afterwards).  Call it before
 * destroying a stream the library has used.  Fails (1) while the stream
 * captures.  topsaten_release_graph_workspace_pool does the same.
 *
 * ubridge_workspace_stats: pool buffers allocated and not yet freed (count,
 * bytes, all devices and streams) and caller-allocator blocks not yet handed
 * back (0 between calls). */
/* ubridge_init: hipBLASLt set-up of the current device, now (outside any
 * capture); optional -- the first eager call does it.  0 = ok. */
int ubridge_init(void);
typedef int (*ubridge_ws_alloc_fn)(void** ptr, size_t bytes, void* stream, void* ctx);
typedef void (*ubridge_ws_free_fn)(void* ptr, void* stream, void* ctx);
int ubridge_set_workspace_allocator(ubridge_ws_alloc_fn alloc, ubridge_ws_free_fn free_fn,
                                    void* ctx);
int ubridge_release_workspace(void* stream);
int ubridge_workspace_stats(size_t* live_buffers, size_t* live_bytes, long* caller_blocks_out);

/* ------------------------------------------------ launch-shape knobs
 * Replaces the host tiling choice of gemm_tuner.rs:326-600 (GEMM_OP_PARAS,
 * :222-258): every launcher picks its MI355X launch shape from the problem
 * shape; a knob set here overrides that rule process-wide (0 = automatic).
 * Knobs: "gemv_lds_rows" (Q4_K LDS GEMV rows per wavefront, 1/2/4; < 0 turns
 * the LDS path off), "gemv_lds_waves" (its wavefronts per workgroup, 4/8),
 * "gemv_rows" / "gemv_iters" (register-path GEMV), "gemm_tile" (1 = 128x128,
 * 2 = 128x256, 3 = 256x256; for the pipelined W4A16 kernel 1 = 128x256 split
 * over K, 3 = 256x256), "gemv_mfma_m" (fewest tokens that take the multi-token
 * MFMA GEMVs for Q8_0 / Q4_K -- the ring GEMV, else the int8-MFMA one; > 16
 * turns them off), "w4a16_path" (any value but 0 also turns off the
 * dequantized-slab + hipBLASLt route of the quantized matmul_* /
 * ubridge_w4a16_gemm: 1 = the generic MFMA core instead of the pipelined
 * W4A16 kernel and of QMatMul's GEMMs; 2 = no decode GEMV for the quantized
 * and dense matmul_* and QMatMul never on the pipelined GEMM; 3 = the
 * pipelined GPTQ kernel's 4-wavefront variant; 4 = QMatMul on the pipelined
 * GEMM at every size from 17 tokens; 5 = GPTQ 256x256 tiles of 8 wavefronts
 * each owning 256x64, for M >= 2048; 6 = the slab route from 17 tokens; 7 =
 * no K split over workgroups in the pipelined GEMMs), "moe_gemm_path"
 * (grouped expert GEMM tile / load-ring variant,
 * 1..9), "gemv_mm" (the 3..16-token ring GEMV for Q4_0 / Q8_0 / Q4_K with K a
 * multiple of 1024: < 0 off, 1..22 a fixed tile / ring variant, taken from 3
 * tokens on), "gemv_persist" (one-launch quantize + GEMV: < 0 one workgroup
 * per row group, > 0 the persistent grid; 2 / 3 force the rolling prefetch
 * of the next row group off / on), "gemv_q80_lds" (one-launch Q4_0 / Q8_0:
 * < 0 register path, > 0 LDS-staged path), "gemv_fuse_m" (most tokens, 1..4,
 * whose activation quantization runs inside the GEMV kernel).  Initial values
 * come from the environment (UBRIDGE_GEMV_LDS, UBRIDGE_GEMV_W,
 * UBRIDGE_GEMV_R, UBRIDGE_GEMV_U, UBRIDGE_GEMM_TILE, UBRIDGE_GEMV_MFMA_M,
 * UBRIDGE_W4A16_PATH, UBRIDGE_MOE_GEMM_PATH, UBRIDGE_GEMV_MM,
 * UBRIDGE_GEMV_PERSIST, UBRIDGE_GEMV_Q80_LDS, UBRIDGE_GEMV_FUSE_M).  Unknown
 * names: error 1. */
int ubridge_tune_set(const char* name, int value);
int ubridge_tune_get(const char* name);

/* ------------------------------------------------- GGUF dequant (module "quant")
 * Input is the reference SoA layout: [nb block headers][nb block payloads].
 *   Q8_0: [nb x fp16 d][nb x 32 int8]                          (kernels/quant.cpp:217-220)
 *   Q4_K: [nb x {fp16 d, fp16 dmin, u8 scales[12]}][nb x 128 B] (kernels/quant.cpp:439-442)
 *   Q4_0: [nb x fp16 d][nb x 16 B], GGML nibble order            (block_q4_0, quant.cpp:64-70)
 * numel must be a multiple of the block size (32 / 256). */
/* replaces dequantize_block_q8_0_{f16,bf16,f32} (kernels/quant.cpp:257-268) */
void dequantize_block_q8_0_f16(const int8_t* in, void* out, size_t numel, void* stream);
void dequantize_block_q8_0_bf16(const int8_t* in, void* out, size_t numel, void* stream);
void dequantize_block_q8_0_f32(const int8_t* in, void* out, size_t numel, void* stream);
/* replaces dequantize_block_q4_k_{f16,bf16,f32} (kernels/quant.cpp:477-488) */
void dequantize_block_q4_k_f16(const int8_t* in, void* out, size_t numel, void* stream);
void dequantize_block_q4_k_bf16(const int8_t* in, void* out, size_t numel, void* stream);
void dequantize_block_q4_k_f32(const int8_t* in, void* out, size_t numel, void* stream);
/* Q4_0 has a block struct but no kernel in the reference (quant.cpp:64-70);
 * same signature as the Q8_0 entry points. */
void dequantize_block_q4_0_f16(const int8_t* in, void* out, size_t numel, void* stream);
void dequantize_block_q4_0_bf16(const int8_t* in, void* out, size_t numel, void* stream);
void dequantize_block_q4_0_f32(const int8_t* in, void* out, size_t numel, void* stream);
/* replaces quantize_block_q8_0_{bf16,f16,f32}(T* in, int8_t* out, size_t
 * input_bytes, size_t output_bytes) (kernels/quant.cpp:331-353); output SoA. */
void quantize_block_q8_0_bf16(const void* in, int8_t* out, size_t in_bytes, size_t out_bytes, void* stream);
void quantize_block_q8_0_f16(const void* in, int8_t* out, size_t in_bytes, size_t out_bytes, void* stream);
void quantize_block_q8_0_f32(const void* in, int8_t* out, size_t in_bytes, size_t out_bytes, void* stream);
/* replaces quantize_block_q4_k_* (kernels/quant.cpp:644-657), whose quantize
 * call is commented out (:639): reports error 3 (unsupported). */
void quantize_block_q4_k_bf16(const void* in, int8_t* out, size_t in_bytes, size_t out_bytes, void* stream);
void quantize_block_q4_k_f16(const void* in, int8_t* out, size_t in_bytes, size_t out_bytes, void* stream);
void quantize_block_q4_k_f32(const void* in, int8_t* out, size_t in_bytes, size_t out_bytes, void* stream);
/* GGUF on-disk AoS blocks <-> the SoA layout above (qtype: GGML id 2 = Q4_0,
 * 8 = Q8_0, 12 = Q4_K).  The reference expects weights already in SoA form
 * (quant.cpp:217-220); this is the loader-side conversion. */
int ubridge_gguf_to_soa(int qtype, const void* aos, void* soa, size_t nblocks, void* stream);
int ubridge_soa_to_gguf(int qtype, const void* soa, void* aos, size_t nblocks, void* stream);

/* ------------------------------------------------ fused decode GEMV (QMatMul)
 * y[M,N] = x[M,K] . W[N,K]^T for W in SoA Q4_0 / Q8_0 / Q4_K, x f32 (0) or
 * bf16 (2), y f32 (0) or bf16 (2).  Replaces the reference's GGUF QMatMul
 * sequence "dequantize_block_* (kernels/quant.cpp:257-268,486-488) then
 * matmul_bf16 (kernels/matmul.cpp:1143-1184)" with one read of the packed
 * weight.  Numerics are Candle's CPU QMatMul method (activations quantized to
 * Q8_0 / Q8_K, integer block dots), run 16 tokens per pass.  Beyond 16
 * tokens ubridge_qmatmul instead computes the reference's GCU sequence (the
 * dequantize_block_*_bf16 values in a bf16 GEMM, f32 accumulate, x rounded
 * to bf16) where that measured faster: Q4_0 and Q8_0 from 17 tokens, Q4_K
 * from 17 (N >= 8192) or 40, and where the GEMM below does not apply from 64
 * (Q4_K) or 40.  Below 768 tokens (K % 256 ==
 * 0, N % 8 == 0): the pipelined MFMA GEMM that dequantizes those values in
 * registers from the packed weight in LDS (K split over workgroups into the
 * per-stream workspace where its grid would leave CUs idle).  Otherwise the weight is dequantized in slabs of up
 * to 256 MB into the per-stream library workspace, each slab a hipBLASLt
 * GEMM; where that cannot run (e.g. first met inside a graph capture) from
 * M = 128 one kernel dequantizing tile by tile in LDS (same values), else
 * the GEMV.  f32 x is converted into the caller's workspace;
 * ubridge_qmatmul_workspace_size includes that room.  The workspace holds the quantized activations; with 1-4
 * tokens (K <= 4096; beyond, Q4_K 1 token, or 2 where K and N are below 8192;
 * Q4_0 / Q8_0 with K % 256 == 0 up to K = 16384 1-4 tokens, 1-2 on rows
 * longer than 8192 of matrices of at most 8192 rows, or 1-2 tokens with
 * K <= 8192 otherwise) ubridge_qmatmul quantizes inside
 * the GEMV kernel instead (one launch, same codes) and leaves it untouched. */
size_t ubridge_qmatmul_workspace_size(int qtype, int M, int K);
int ubridge_quantize_activations(int qtype, const void* x, int x_dtype, int M, int K,
                                 void* workspace, size_t ws_bytes, void* stream);
int ubridge_qmatmul_prequantized(int qtype, const void* w, void* y, int y_dtype, int M, int N,
                                 int K, const void* workspace, void* stream);
int ubridge_qmatmul(int qtype, const void* w, const void* x, int x_dtype, void* y, int y_dtype,
                    int M, int N, int K, void* workspace, size_t ws_bytes, void* stream);
/* No counterpart in the reference.  For callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): ubridge_qmatmul with its workspace in a static per-device
 * array of ubridge_qmatmul_noalloc_max_workspace() bytes (4 MiB) instead of
 * a caller buffer.  Allocates nothing: at prefill sizes it runs the
 * pipelined GEMM without the K split (from 64 tokens for Q4_K, 40 for Q4_0 /
 * Q8_0; other shapes
 * the GEMM that dequantizes in LDS, from 128), never the slab + hipBLASLt form (where
 * ubridge_qmatmul takes that, results differ by summation order, ~1e-3).  Sizes whose
 * workspace on these routes (the quantized activations; from 64 (Q4_K) / 40
 * tokens room for a bf16 copy of f32 x) exceeds the array are rejected
 * (error 1).
 * All calls on one GPU share the array: calls that overlap on one GPU
 * (unordered streams) race. */
size_t ubridge_qmatmul_noalloc_max_workspace(void);
int ubridge_qmatmul_noalloc(int qtype, const void* w, const void* x, int x_dtype, void* y,
                            int y_dtype, int M, int N, int K, void* stream);

/* ------------------------------------------------ weight-only GEMM (module "matmul")
 * The 17 shared arguments of the reference's matmul signature
 * (kernels/matmul.cpp:1143-1215): input_dtype, batch, m, k, n, lhs/rhs/batch
 * multicore flags, lhs_transpose, rhs_transpose, alpha, beta, addmm_beta,
 * sip_m, sip_k, sip_n, broadcasted_weight.  A (sip_m, sip_n) pair naming one
 * of this library's tiles (128x128, 128x256, 256x256, as
 * ubridge_get_gemm_launch_params returns) selects that tile; other values
 * leave the choice to the shape rule; lhs_transpose reports error 3. */
#define UBRIDGE_REF_MM_ARGS                                                             \
  int input_dtype, int batch, int m, int k, int n, int lhs_multicore, int rhs_multicore, \
      int batch_multicore, int lhs_transpose, int rhs_transpose, float alpha, float beta, \
      float addmm_beta, int sip_m, int sip_k, int sip_n, int broadcasted_weight
/* GEMM launch parameters: the #[repr(C)] GEMM_OP_PARAS of src/gemm_tuner.rs:
 * 222-258, field for field (22 int32, 5 float, 6 int32: 132 bytes). */
typedef struct UbridgeGemmOpParas {
  int32_t input_dtype, output_dtype, csb_batch, sip_batch, lhs_csb_k, rhs_csb_k, lhs_csb_m,
      rhs_csb_n, sip_m, sip_k, sip_n, batch_multicore, lhs_multicore, rhs_multicore,
      lhs_pingpong, rhs_pingpong, sdma_lhs_pingpong, sdma_rhs_pingpong, rhs_repeat_copy,
      lhs_transpose, rhs_transpose, out_transpose;
  float alpha, beta, addmm_beta, coef, act_mode;
  int32_t bias, act_en, input_batch, input_m, input_k, input_n;
} UbridgeGemmOpParas;
/* replaces GcuDevice::get_gemm_launch_params (src/gcu_device.rs:185-198) and
 * its per-shape cache AtenGemmTuner::tuner (src/gemm_tuner.rs:326-359):
 * datatype / weight_type are the reference's DATATYPE codes (src/lib.rs:88-106:
 * DataI8 = 0, DataFp16 = 4, DataBf16 = 5, DataI4 = 15).  Returns a pointer to
 * the cached parameters (valid for the life of the process), NULL on an
 * unsupported type (error 3) or shape (error 1).  sip_m x sip_n is the output
 * tile this library launches for the shape; passing the returned sip_m /
 * sip_k / sip_n and *_multicore fields to matmul_* selects that tile. */
const UbridgeGemmOpParas* ubridge_get_gemm_launch_params(int datatype, int weight_type, size_t b,
                                                         size_t m, size_t k, size_t n,
                                                         int rhs_trans);
/* replaces matmul_{bf16,f16}_4bit (kernels/matmul.cpp:1211-1212): b uint8
 * [K/2, N] (low nibble = even k), scales / zeros T [K/g, N],
 * w = T(((float)q - z) * s); rhs_transpose reports error 3. */
void matmul_bf16_4bit(const void* a, const uint8_t* b, void* out, const void* scales,
                      const void* zeros, UBRIDGE_REF_MM_ARGS, int group_size, void* stream);
void matmul_f16_4bit(const void* a, const uint8_t* b, void* out, const void* scales,
                     const void* zeros, UBRIDGE_REF_MM_ARGS, int group_size, void* stream);
/* replaces matmul_{bf16,f16}_8bit (kernels/matmul.cpp:1214-1215): b int8
 * [K, N] or [N, K] (rhs_transpose), scales T per group; zeros unused. */
void matmul_bf16_8bit(const void* a, const int8_t* b, void* out, const void* scales,
                      const void* zeros, UBRIDGE_REF_MM_ARGS, int group_size, void* stream);
void matmul_f16_8bit(const void* a, const int8_t* b, void* out, const void* scales,
                     const void* zeros, UBRIDGE_REF_MM_ARGS, int group_size, void* stream);
/* replaces dense matmul_{bf16,f16} (kernels/matmul.cpp:1181-1184). */
void matmul_bf16(const void* a, const void* b, void* out, UBRIDGE_REF_MM_ARGS, void* stream);
void matmul_f16(const void* a, const void* b, void* out, UBRIDGE_REF_MM_ARGS, void* stream);
/* replaces dequant_{f16,bf16} (kernels/dequant_host.cpp:298-307, declared
 * src/ffi.rs:70-93): rhs uint8 [K, N] packs rows 2k (low nibble) and 2k+1,
 * scale / zeros T [2K/g, N], out T [2K, N]; weight_transpose reports error 3. */
void dequant_bf16(void* out, const uint8_t* rhs, const void* scale, const void* zeros, int K,
                  int N, int weight_transpose, int group_size, void* stream);
void dequant_f16(void* out, const uint8_t* rhs, const void* scale, const void* zeros, int K,
                 int N, int weight_transpose, int group_size, void* stream);
/* W4A16 in the GPTQ layout (no reference counterpart; the reference's 4-bit
 * path is matmul_*_4bit above): qw int32 [K/8, N], scales T [K/g, N],
 * qzeros int32 [K/g, N/8], out T [M, N]; dtype 1 = f16, 2 = bf16. */
int ubridge_w4a16_gemm(const void* a, const int32_t* qw, const void* scales,
                       const int32_t* qzeros, void* out, int M, int K, int N, int group,
                       int dtype, void* stream);
/* Dense GEMM on the same core: w [K, N] (w_transposed = 0) or [N, K]. */
int ubridge_gemm_dense(const void* a, const void* w, void* out, int M, int K, int N,
                       int w_transposed, int dtype, void* stream);

/* ------------------------------------------------ fp8 W8A8 GEMM
 * out[M,N] bf16 = (a[M,K] e4m3 . w_nk[N,K]^T e4m3) * sa[M] * sw[N].  No
 * reference counterpart in kernels/ (the reference's fp8 path is the
 * topsaten library wrapper, kernels/topsaten_ops_wrapper.cpp).  By default
 * hipBLASLt's fp8 GEMM with row / column scale vectors where it serves the
 * shape (set up at the first call outside graph capture, or by
 * ubridge_init), else the library's own MFMA kernel; tuning knob gemm_tile
 * 2 / 3 / 4 forces the own kernels. */
int ubridge_fp8_gemm(const uint8_t* a, const float* sa, const uint8_t* w_nk, const float* sw,
                     void* out, int M, int K, int N, void* stream);
int ubridge_fp8_transpose(const uint8_t* in, uint8_t* out, int R, int C, void* stream);
/* x [R, C] (x_dtype 0 f32, 1 f16, 2 bf16) -> e4m3 q with scale[r] = amax / 448
 * (1 for an all-zero row). */
int ubridge_fp8_quantize_rows(const void* x, int x_dtype, uint8_t* q, float* scale, int R,
                              int C, void* stream);

/* ------------------------------------------------ fused MoE
 * replaces topk_softmax_{f32,f16,bf16} (kernels/topk_softmax_host.cpp:178-209,
 * src/ffi.rs:205-236); E <= 4096, k <= min(E, 64). */
void topk_softmax_f32(const float* in, float* out, int* idx, int T, int E, int k, int norm,
                      void* stream);
void topk_softmax_f16(const void* in, void* out, int* idx, int T, int E, int k, int norm,
                      void* stream);
void topk_softmax_bf16(const void* in, void* out, int* idx, int T, int E, int k, int norm,
                       void* stream);
/* replaces moe_align_block_size (kernels/moe_align_host.cpp:923, src/ffi.rs:
 * 149-161); num_experts <= 1024.  Out-of-range expert ids raise the device
 * flag read by ubridge_device_error instead of trapping. */
void moe_align_block_size(int* sorted_ids, int* experts_ids, int* num_tokens_post_pad,
                          const int* topk_ids, const int* real_token_num, const int* expert_map,
                          int num_experts, int block_size, int token_num, int topk, void* stream);
/* replaces invoke_fused_moe_{f16,bf16} (kernels/fused_moe_host.cpp:504-537,
 * src/ffi.rs:163-203): C [M*top_k, N] = A[token] . B[expert]^T, B T [E, N, K]. */
void invoke_fused_moe_bf16(void* C, const void* A, const void* B, const void* bias,
                           const float* topk_weights, const int* sorted_ids,
                           const int* experts_ids, const int* num_tokens_post_pad, int M, int K,
                           int N, int E, int topk_ids_size, int top_k, int block_size,
                           int mul_routed_weight, int bias_flag, void* stream);
void invoke_fused_moe_f16(void* C, const void* A, const void* B, const void* bias,
                          const float* topk_weights, const int* sorted_ids,
                          const int* experts_ids, const int* num_tokens_post_pad, int M, int K,
                          int N, int E, int topk_ids_size, int top_k, int block_size,
                          int mul_routed_weight, int bias_flag, void* stream);
/* Same with int8 experts B [E, N, K] and per-output-channel scales
 * B_scale T [E, N] (no reference counterpart). */
int ubridge_fused_moe_w8a16(void* C, const void* A, const int8_t* B, const void* B_scale,
                            const void* bias, const float* topk_weights, const int* sorted_ids,
                            const int* experts_ids, const int* num_tokens_post_pad, int M, int K,
                            int N, int E, int topk_ids_size, int top_k, int block_size,
                            int mul_routed_weight, int bias_flag, int dtype, void* stream);
/* ubridge_fused_moe_w8a16 (the down expert GEMM) followed by the top-k
 * combine in one call (the reference's combine after the second expert
 * GEMM, fused_moe_host.cpp:420-427 / moe_host.cpp:27-93): C as
 * ubridge_fused_moe_w8a16 writes it, plus Y [topk_ids_size / top_k, N] =
 * T(sum over j of C[t * top_k + j, :]) in slot order with f32 accumulation,
 * the bits of ubridge_moe_sum.  Two launches on the stream. */
int ubridge_fused_moe_w8a16_combine(void* Y, void* C, const void* A, const int8_t* B,
                                    const void* B_scale, const void* bias,
                                    const float* topk_weights, const int* sorted_ids,
                                    const int* experts_ids, const int* num_tokens_post_pad, int M,
                                    int K, int N, int E, int topk_ids_size, int top_k,
                                    int block_size, int mul_routed_weight, int bias_flag,
                                    int dtype, void* stream);
/* topk_softmax_{dtype} + moe_align_block_size (no expert_map /
 * real_token_num) in one call: the routing before the grouped GEMM (the
 * reference's topk_softmax_host.cpp:103-208 and moe_align_host.cpp:51-935).
 * Outputs are those of the two operators; topk_w_f32 (nullable) also
 * receives the f32 value of every final weight, the GEMM's topk_weights
 * operand, so no conversion launch is needed.  E <= 1024. */
int ubridge_moe_route(const void* logits, int dtype, void* topk_w, float* topk_w_f32,
                      int* topk_ids, int* sorted_ids, int* experts_ids,
                      int* num_tokens_post_pad, int T, int E, int k, int renormalize,
                      int block_size, void* stream);
/* Gate/up expert GEMM with silu_and_mul fused into the epilogue (no
 * counterpart in the reference, which runs invoke_fused_moe then
 * silu_and_mul, fused_moe_host.cpp:43-252 / topsaten_ops_wrapper.cpp:375-391):
 * B int8 [E, N, K] holds the gate rows [0, N/2) and up rows [N/2, N);
 * C [topk_ids_size, N/2] = T(silu(g) * u) of the T-rounded GEMM outputs, the
 * same values as the two-call sequence.  Arguments as ubridge_fused_moe_w8a16
 * without the routed weight. */
int ubridge_fused_moe_w8a16_silu(void* C, const void* A, const int8_t* B, const void* B_scale,
                                 const void* bias, const int* sorted_ids, const int* experts_ids,
                                 const int* num_tokens_post_pad, int M, int K, int N, int E,
                                 int topk_ids_size, int top_k, int block_size, int bias_flag,
                                 int dtype, void* stream);

/* out[T, d] = silu(x[T, :d]) * x[T, d:] and out[T, N] = sum_k in[T, k, N]:
 * the activation and combine steps between the two expert GEMMs. */
int ubridge_silu_and_mul(void* out, const void* x, int T, int d, int dtype, void* stream);
int ubridge_moe_sum(void* out, const void* in, int T, int k, int N, int dtype, void* stream);
/* Status-returning MoE trio: replace topsaten_topk_softmax_f32,
 * topsaten_moe_align_block_size, topsaten_fused_moe_gemm and
 * topsaten_release_graph_workspace_pool (kernels/topsaten_moe_wrapper.cpp:80,
 * 108, 152, 214; src/ffi.rs:671-715).  Same arguments; 0 on success, else
 * the ubridge_last_error code.  token_expert_indices[t, j] = j * num_tokens
 * + t.  fused_moe_gemm: C [num_tokens, topk, inter_dim], A [num_tokens,
 * hidden_dim] (slot t * topk + j reads row t, with or without
 * mul_routed_weight), B [num_experts, inter_dim, hidden_dim], dtype_code 4 fp16 /
 * 5 bf16 (8 fp32 returns 3, unsupported); topk_ids is not read.  The three
 * allocate nothing; the release hook frees the stream's library pool
 * (ubridge_release_workspace). */
int topsaten_topk_softmax_f32(float* gating_output, float* topk_weights, int32_t* topk_indices,
                              int32_t* token_expert_indices, int32_t num_tokens,
                              int32_t num_experts, int32_t topk, int32_t norm_topk_prob,
                              void* stream);
int topsaten_moe_align_block_size(int32_t* sorted_token_ids, int32_t* experts_ids,
                                  int32_t* num_tokens_post_pad, int32_t* topk_ids,
                                  int32_t num_tokens, int32_t topk, int32_t num_experts,
                                  int32_t block_size, void* stream);
int topsaten_fused_moe_gemm(void* c_ptr, void* a_ptr, void* b_ptr, float* topk_weights,
                            int32_t* topk_ids, int32_t* sorted_token_ids, int32_t* expert_ids,
                            int32_t* num_tokens_post_padded, int32_t mul_routed_weight,
                            int32_t topk_val, int32_t block_size, int32_t num_tokens,
                            int32_t hidden_dim, int32_t inter_dim, int32_t num_experts,
                            int32_t dtype_code, void* stream);
void topsaten_release_graph_workspace_pool(void* stream);
/* replace moe_{f16,bf16} and indexed_moe_{f16,bf16} (kernels/moe_host.cpp:84,
 * 279; src/ffi.rs:44-69,121-148). */
void moe_bf16(void* y, const void* e_out, const float* w, const uint32_t* idx,
              const uint32_t* top, int N, int K, int M, int topk, void* stream);
void moe_f16(void* y, const void* e_out, const float* w, const uint32_t* idx,
             const uint32_t* top, int N, int K, int M, int topk, void* stream);
void indexed_moe_bf16(const void* in, const void* w, void* out, const uint32_t* idx, int N,
                      int K, int M, int batch, int topk, int num_experts, void* stream);
void indexed_moe_f16(const void* in, const void* w, void* out, const uint32_t* idx, int N,
                     int K, int M, int batch, int topk, int num_experts, void* stream);
/* Synchronizes `stream`, returns and clears the device-side index-error flag
 * (4) raised by moe_align_block_size / the MoE GEMMs. */
int ubridge_device_error(void* stream);

/* ------------------------------------------------ name-keyed kernel launch
 * Replaces GcuDevice::get_or_load_func(func, module) (src/gcu_device.rs:160-183,
 * DeviceExecutor::get_function src/device_executor.rs:523-531) and
 * GcuLaunchAsync::launch (src/gcu_launch.rs:121-181): `args[i]` points at the
 * i-th positional argument of the reference kernel signature; the stream is
 * appended by the library.  Unknown names return NULL (the reference returned
 * a silent no-op function). */
const void* ubridge_get_function(const char* name, const char* module);
int ubridge_has_function(const char* name);   /* DeviceExecutor::has_function, :533-538 */
int ubridge_num_functions(void);
const char* ubridge_function_name(int i);
int ubridge_launch(const void* function, void** args, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* UBRIDGE_HIP_H */
