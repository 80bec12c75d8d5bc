// lds_dma.h -- direct-to-LDS buffer loads for the pipelined MFMA kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef unsigned int ub_u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kDmaOOB = 0x80000000u;  // an offset past every buffer: reads zero

// Raw buffer descriptor (base, byte size, 32-bit raw format) in SGPRs.
__device__ __forceinline__ ub_u32x4 ub_desc(const void* base, uint64_t bytes) {
  const uint32_t n = bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes;
  const uint64_t p = (uint64_t)base;
  ub_u32x4 d;
  d.x = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)p);
  d.y = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  d.z = (uint32_t)__builtin_amdgcn_readfirstlane(n);
  d.w = 0x00020000u;
  return d;
}

// Direct-to-LDS load: lane i's 16 bytes at byte offset `off` of the buffer
// land at lds + 16 i (out-of-range offsets write zeros).  Written as inline
// asm so that the compiler does not treat it as an LDS store: it would
// otherwise wait for every outstanding one before any LDS read, including
// the loads of pipeline stages still in flight.  Callers wait for these
// loads explicitly (s_waitcnt vmcnt).  An M0 write needs one wait state
// before the LDS DMA that reads it: s_nop 0.  M0 is listed as clobbered (the
// compiler warns that it is reserved): kernels using this must not rely on
// M0 otherwise -- no LDS-DMA builtins, GWS or s_movrel -- which holds for
// the kernels of this library (their assembly sets M0 only here).
__device__ __forceinline__ void ub_lds_load16(const ub_u32x4& d, void* lds, uint32_t off) {
  const uint32_t la = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds;
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(la)), "v"(off), "s"(d)
               : "memory", "m0");
}

// The same with a scalar offset added to every lane's: lane i's 16 bytes at
// voff + soff land at LDS address lds + 16 i (lds a 32-bit LDS address).  A
// K-loop passes its step's byte offset as soff, so per-lane offsets are set
// up once.
__device__ __forceinline__ void ub_lds_load16_at(const ub_u32x4& d, uint32_t lds, uint32_t voff,
                                                 uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(d),
                 "s"(__builtin_amdgcn_readfirstlane(soff))
               : "memory", "m0");
}

// The same with the non-temporal hint (nt): for data read once, such as
// streamed weights.
__device__ __forceinline__ void ub_lds_load16_at_nt(const ub_u32x4& d, uint32_t lds,
                                                    uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(d),
                 "s"(__builtin_amdgcn_readfirstlane(soff))
               : "memory", "m0");
}

// 4-byte form: lane i's dword at voff + soff lands at LDS address lds + 4 i.
__device__ __forceinline__ void ub_lds_load4_at(const ub_u32x4& d, uint32_t lds, uint32_t voff,
                                                uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(d),
                 "s"(__builtin_amdgcn_readfirstlane(soff))
               : "memory", "m0");
}

// LDS reads by 32-bit LDS address.
typedef unsigned int ub_v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ub_lds_read16(uint32_t a) {
  const ub_v4u v = *(const __attribute__((address_space(3))) ub_v4u*)(size_t)a;
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ub_lds_read8(uint32_t a) {
  typedef unsigned int v2u __attribute__((ext_vector_type(2)));
  const v2u v = *(const __attribute__((address_space(3))) v2u*)(size_t)a;
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ub_lds_read4(uint32_t a) {
  return *(const __attribute__((address_space(3))) uint32_t*)(size_t)a;
}
__device__ __forceinline__ uint32_t ub_lds_read2(uint32_t a) {
  return *(const __attribute__((address_space(3))) uint16_t*)(size_t)a;
}
template <class T>
__device__ __forceinline__ uint32_t ub_lds_addr(T* p) {
  return (uint32_t)(size_t)(__attribute__((address_space(3))) T*)p;
}

// s_waitcnt vmcnt(n) for a compile-time n <= 63 (gfx9 encoding: vmcnt bits
// 3:0 and 15:14; expcnt / lgkmcnt left at their maximum), fenced against
// compiler reordering.
template <int N>
__device__ __forceinline__ void ub_wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt immediate");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
  __builtin_amdgcn_sched_barrier(0);
}

// Workgroup barrier that does not wait for outstanding vector-memory loads
// (__syncthreads() would also drain the pipeline's in-flight stages).  LDS
// reads issued before it have been consumed by the caller, so they are done.
__device__ __forceinline__ void ub_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Tile order for a 1-D grid of tm x tn output tiles.  The hardware hands
// workgroup i to XCD i % 8, each XCD with its own L2, so ids are first
// regrouped so every XCD gets one contiguous run of the order; the order
// itself walks groups of `gm` tile rows column by column, so the tiles
// resident at one time share a few A row-panels and B column-panels
// instead of sweeping whole rows of B.
__device__ __forceinline__ void ub_tile_order(int tm, int tn, int gm, int& im, int& in_) {
  const int total = tm * tn;
  int pid = blockIdx.x;
  constexpr int kXcd = 8;
  if (total % kXcd == 0) pid = (pid % kXcd) * (total / kXcd) + pid / kXcd;
  const int per_group = gm * tn;
  const int g = pid / per_group, first = g * gm;
  const int rows = min(gm, tm - first);
  const int r = pid % per_group;
  im = first + r % rows;
  in_ = r / rows;
}
