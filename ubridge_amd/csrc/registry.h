// registry.h -- argument-array thunks for the name-keyed launch table.
// Each thunk reads args[i] as a pointer to the i-th positional argument of
// the reference kernel signature, exactly as GcuLaunchAsync passes them
// (src/gcu_launch.rs:192, as_kernel_param).
#pragma once
#include <stddef.h>
#include <stdint.h>

extern "C" int ubridge_last_error(void);
extern "C" const char* ubridge_last_error_string(void);

typedef void (*ub_thunk)(void** args, void* stream);

#define UB_ARG(T, i) (*(T*)args[i])

// module, name for every launchable kernel.
#define UB_REGISTRY_ENTRIES(X)                 \
  X("quant", dequantize_block_q8_0_f16)        \
  X("quant", dequantize_block_q8_0_bf16)       \
  X("quant", dequantize_block_q8_0_f32)        \
  X("quant", dequantize_block_q4_k_f16)        \
  X("quant", dequantize_block_q4_k_bf16)       \
  X("quant", dequantize_block_q4_k_f32)        \
  X("quant", dequantize_block_q4_0_f16)        \
  X("quant", dequantize_block_q4_0_bf16)       \
  X("quant", dequantize_block_q4_0_f32)        \
  X("quant", quantize_block_q8_0_f16)          \
  X("quant", quantize_block_q8_0_bf16)         \
  X("quant", quantize_block_q8_0_f32)          \
  X("quant", quantize_block_q4_k_f16)          \
  X("quant", quantize_block_q4_k_bf16)         \
  X("quant", quantize_block_q4_k_f32)          \
  X("matmul", matmul_bf16_4bit)                \
  X("matmul", matmul_f16_4bit)                 \
  X("matmul", matmul_bf16_8bit)                \
  X("matmul", matmul_f16_8bit)                 \
  X("matmul", matmul_bf16)                     \
  X("matmul", matmul_f16)

#define UB_DECL_THUNK(mod, nm) void ub_thunk_##nm(void** args, void* stream);
UB_REGISTRY_ENTRIES(UB_DECL_THUNK)
#undef UB_DECL_THUNK
