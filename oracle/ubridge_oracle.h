/*
 * ubridge_oracle.h -- CPU restatement of Ubridge's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product path (ubridge_amd + libubridge_hip.so) never calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the EnflameTechnology/Ubridge tree) or, where the
 * reference has no kernel, the published GGML / Candle method it follows.
 *
 * Pinning status (what checks each function; see tests/test_oracle_*.py):
 *   fp16/bf16/e4m3 conversions ... exhaustive / closed form vs numpy + torch
 *   dequant q8_0 / q4_0 / q4_k ... independent numpy restatement (golden
 *                                  fixtures) + closed-form special cases
 *   quantize q8_0 / q8_k ......... golden fixtures + invariants
 *   qmatmul (Candle CPU method) .. exact-representable activations reduce it
 *                                  to an f64 dense dot; bound vs f64 otherwise
 *   w8a16 / w4a16 / fp8 gemm ..... brute force f64 on the decoded weights
 *   topk_softmax ................. numpy softmax + argsort, tie rule cases
 *   moe_align_block_size ......... permutation / padding invariants + numpy
 *   fused_moe .................... per-slot dense recomputation
 *   moe_combine .................. closed forms (w = 1 / w = 0 / duplicate
 *                                  rows accumulate in slot order) vs numpy
 *   indexed_moe .................. integer-valued inputs (exact f32 sums)
 *                                  vs numpy int64; numpy f32 loop otherwise
 * The reference's own tests hold no golden vectors for this path, and the
 * reference cannot be built here (TopsCC + closed acore library), so no
 * function is pinned against reference *outputs*.
 */
#ifndef UBRIDGE_ORACLE_H
#define UBRIDGE_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 2 };
/* GGML type ids */
enum { ORC_Q4_0 = 2, ORC_Q8_0 = 8, ORC_Q4_K = 12 };

/* ---- scalar conversions (IEEE round-to-nearest-even) ---- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
float orc_e4m3_to_f32(uint8_t v);
uint8_t orc_f32_to_e4m3(float f); /* saturating, RNE, OCP e4m3fn */
void orc_f32_to_bf16_n(const float* in, uint16_t* out, size_t n);
void orc_bf16_to_f32_n(const uint16_t* in, float* out, size_t n);

/* ---- GGUF block dequant, reference SoA layout "[scales...][data...]" ---- */
void orc_dequant_q8_0(const uint8_t* in, void* out, size_t numel, int out_dtype);
void orc_dequant_q4_0(const uint8_t* in, void* out, size_t numel, int out_dtype);
void orc_dequant_q4_k(const uint8_t* in, void* out, size_t numel, int out_dtype);

/* AoS (GGUF on-disk) <-> SoA repack; nblocks blocks. */
void orc_aos_to_soa(int qtype, const uint8_t* aos, uint8_t* soa, size_t nblocks);
void orc_soa_to_aos(int qtype, const uint8_t* soa, uint8_t* aos, size_t nblocks);

/* ---- activation-side quantization (Candle from_float) ---- */
/* Q8_0 in SoA layout: [nb x fp16 d][nb x 32 int8]; n multiple of 32. */
void orc_quantize_q8_0(const float* x, size_t n, uint8_t* soa_out);
/* Q8_K: per 256 elements f32 d, 256 int8, 16 int16 bsums. */
void orc_quantize_q8_k(const float* x, size_t n, float* d, int8_t* qs, int16_t* bsums);

/* ---- Candle CPU QMatMul: y[M,N] = x[M,K] . W[N,K]^T ---- */
void orc_qmatmul(int qtype, const uint8_t* w_soa, const float* x, float* y,
                 int M, int N, int K, int nthreads);

/* ---- W8A16 / W4A16 GEMM (bf16 activations, f32 accumulate, bf16 out) ---- */
/* w8: int8 [K,N] (rhs_t=0) or [N,K] (rhs_t=1); scales bf16 [K/g, N]; g<=0 -> K */
void orc_w8a16_gemm(const uint16_t* a, const int8_t* w, const uint16_t* scales,
                    uint16_t* out, int M, int K, int N, int group, int rhs_t);
/* GPTQ-style: qw int32 [K/8, N] (8 K-consecutive nibbles, LSB first),
 * scales bf16 [K/g, N], zeros int32 [K/g, N/8] (8 N-consecutive nibbles). */
void orc_w4a16_dequant(const int32_t* qw, const uint16_t* scales, const int32_t* qz,
                       uint16_t* wout /* bf16 [K,N] */, int K, int N, int group);
void orc_w4a16_gemm(const uint16_t* a, const int32_t* qw, const uint16_t* scales,
                    const int32_t* qz, uint16_t* out, int M, int K, int N, int group,
                    int nthreads);
/* reference-layout 4-bit dequant (dequant_host.cpp): rhs u8 [K,N] packed rows,
 * out [2K, N]; scale/zeros T [2K/g, N]; w = (q - zero) * scale. */
void orc_dequant_u4_ref(const uint8_t* rhs, const uint16_t* scale, const uint16_t* zeros,
                        uint16_t* out, int K, int N, int group, int dtype);

/* ---- fp8 W8A8 ---- */
void orc_fp8_quantize_rows(const float* x, uint8_t* q, float* scale, int R, int C);
void orc_fp8_gemm(const uint8_t* a, const float* sa, const uint8_t* w, const float* sw,
                  uint16_t* out, int M, int K, int N, int nthreads);

/* ---- MoE routing + grouped GEMM ---- */
void orc_topk_softmax(const void* in, void* out, int32_t* idx, int T, int E, int k,
                      int norm, int dtype);
/* returns num_tokens_post_pad; sorted_ids sized T*k + E*(bs-1). */
int orc_moe_align_block_size(int32_t* sorted_ids, int32_t* experts_ids, int32_t* ntpp,
                             const int32_t* topk_ids, const int32_t* real_token_num,
                             const int32_t* expert_map, int E, int bs, int T, int k);
/* fused MoE: B is [E,N,K]; bf16 (wq==NULL) or int8 + per-channel bf16 scales [E,N]. */
void orc_fused_moe(uint16_t* C, const uint16_t* A, const uint16_t* B, const int8_t* Bq,
                   const uint16_t* Bscale, const uint16_t* bias, const float* topk_w,
                   const int32_t* sorted_ids, const int32_t* experts_ids,
                   const int32_t* ntpp, int M, int K, int N, int E, int topk_ids_size,
                   int top_k, int bs, int mul_routed_weight, int bias_flag, int nthreads);

#ifdef __cplusplus
}
/* Legacy MoE combine, moe_{f16,bf16} (kernels/moe_host.cpp:27-93): for each
 * k in order, if idx[k] < N and top[k] < topk,
 *   y[idx[k], :] = T(y[idx[k], :] + T(e_out[k, :] * w[idx[k] * topk + top[k]])).
 * dt: 1 = f16, 2 = bf16. */
void orc_moe_combine(int dt, uint16_t* y, const uint16_t* e_out, const float* w,
                     const uint32_t* idx, const uint32_t* top, int N, int K, int M, int topk);
/* indexed_moe_{f16,bf16} (kernels/moe_host.cpp:118-293): for b < batch,
 * i < topk with e = idx[b * topk + i] < E,
 *   out[b, i, :] = T(W[e] (N x K) . in[b, M == 1 ? 0 : i, :])   (moe_host.cpp:168)
 * accumulated in f32 with k in order, each product and sum rounded on its own
 * (the reference's CPU check moe_matmul, :325-355), then rounded to T; pairs with e >= E are
 * left untouched (the decode kernel's write sits inside the expert check,
 * :255-270). */
void orc_indexed_moe(int dt, const uint16_t* in, const uint16_t* w, uint16_t* out,
                     const uint32_t* idx, int N, int K, int M, int batch, int topk, int E);
#endif
#endif
