/*
 * ubridge_hip.h -- C ABI of libubridge_hip.so, the MI355X (gfx950) drop-in
 * for Ubridge's quantized-matmul path.
 *
 * Conventions shared by every entry point:
 *   - All pointers are device pointers the caller allocated; the library
 *     allocates nothing on these paths.
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
 * Q8_0 / Q8_K, integer block dots).  Efficient for M <= 16; larger M runs
 * in chunks of 16.  The workspace holds the quantized activations. */
size_t ubridge_qmatmul_workspace_size(int qtype, int M, int K);
int ubridge_quantize_activations(int qtype, const void* x, int x_dtype, int M, int K,
                                 void* workspace, size_t ws_bytes, void* stream);
int ubridge_qmatmul_prequantized(int qtype, const void* w, void* y, int y_dtype, int M, int N,
                                 int K, const void* workspace, void* stream);
int ubridge_qmatmul(int qtype, const void* w, const void* x, int x_dtype, void* y, int y_dtype,
                    int M, int N, int K, void* workspace, size_t ws_bytes, void* stream);

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
