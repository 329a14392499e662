// Device helpers shared by the gfx950 kernels: vector types, raw buffer descriptors, direct-to-LDS
// loads (buffer_load_dwordx4 ... lds / global_load_lds_dwordx4) and the vmcnt wait.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mmm {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef __fp16 fp16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

#define LDS_AS __attribute__((address_space(3)))

// Buffer descriptor word 3 for gfx9-family raw buffers (32-bit data format, no swizzle).
constexpr int kRsrcWord3 = 0x00020000;
// Byte offset used for masked-off chunks; every descriptor's range is clipped below it.
constexpr uint32_t kOobOffset = 0x7ffffff0u;

// Eight zero halves in global memory (one copy per source file), never written.  The element
// gathers load an element past an operand's edge from here instead of masking the loaded value:
// a value that a later select may discard lets the compiler sink its load into a branch of its
// own, whose wait then holds back every load after it (one memory round trip per element).
static __device__ __attribute__((aligned(16))) _Float16 kZeroHalves[8];

// Raw buffer descriptor (base, num_records bytes, word 3) built from uniform values.
__device__ __forceinline__ i32x4 make_rsrc(const void* base, uint32_t num_records) {
  const uint64_t b = (uint64_t)(uintptr_t)base;
  return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)b), __builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32)),
               __builtin_amdgcn_readfirstlane((int)num_records), kRsrcWord3};
}

// A buffer descriptor's record count for `bytes` readable bytes: 0 if none, at most kOobOffset.
__device__ __forceinline__ uint32_t clip_records(int64_t bytes) {
  if (bytes <= 0) return 0u;
  return bytes > (int64_t)kOobOffset ? kOobOffset : (uint32_t)bytes;
}

__device__ __forceinline__ uint32_t lds_addr_of(const char LDS_AS* p) { return (uint32_t)(uintptr_t)p; }

// 16 bytes per lane from the buffer at byte offset voff straight into LDS at
// lds_addr + 16 * lane (buffer_load_dwordx4 ... lds; m0 holds the wave's LDS base).
// Issued as inline asm so the compiler does not treat every later LDS read as dependent on
// it: completion is awaited explicitly (wait_vmcnt) before the LDS is read.  Out-of-range
// offsets (>= num_records) write zeros.  DS instructions on gfx9-family targets do not read
// m0, so overwriting it here is safe.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_b128(uint32_t lds_addr, i32x4 rsrc, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(rsrc)
               : "memory", "m0");
}
// The same load with the non-temporal policy, for an operand streamed once from HBM: its lines
// are not kept in the caches for reuse, so the stream does not evict what the next lines need.
__device__ __forceinline__ void dma_b128_nt(uint32_t lds_addr, i32x4 rsrc, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(rsrc)
               : "memory", "m0");
}
// The same 16 bytes per lane from a 64-bit global address (global_load_lds_dwordx4, gfx950),
// for operands whose per-lane offsets do not fit a buffer's 32 bits.  No range check: the
// caller passes addresses inside the operand.
__device__ __forceinline__ void dma_b128_flat(uint32_t lds_addr, const void* src) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds_addr), "v"(src)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Wait until at most N of this wave's vector-memory operations are outstanding (they
// complete in issue order), i.e. all but the N most recent loads have landed.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass checks "I" against its own (narrower) range
  asm volatile("s_waitcnt vmcnt(%0)" ::"I"(N) : "memory");
#endif
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

}  // namespace mmm
