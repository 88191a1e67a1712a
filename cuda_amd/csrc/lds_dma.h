// HBM -> LDS direct loads and hand-issued LDS reads for gfx950.
//
// global_load_lds_dwordx4 moves 16 bytes per lane from global memory straight
// into LDS (lane l's bytes land at the wave-uniform destination + 16 * l), so
// bytes in flight cost no VGPRs and no ds_write. The compiler's own
// wait-for-everything before LDS reads that might alias such a load would
// serialise a multi-stage ring, so the kernels read LDS with hand-issued
// ds_read instructions (inline asm the compiler does not treat as LDS
// accesses) and wait on the counters explicitly:
//   s_waitcnt vmcnt(N)    - all but the N most recent vector-memory loads done
//   s_waitcnt lgkmcnt(N)  - all but the N most recent LDS reads done
// and `after_wait(x)` re-defines a read's result after its wait so that no
// use of it can be scheduled above the wait.
#pragma once

#include "common.h"

namespace ca {

__device__ __forceinline__ uint32_t lds_off(const void* p) {
  return (uint32_t)(uintptr_t)(const CA_LDS void*)p;
}

// The LDS reads and waits are gfx950 instructions; the host pass of the HIP
// compiler (which also parses device code) gets inert stand-ins.
#if __HIP_DEVICE_COMPILE__
#define CA_DEVICE_ASM(...) asm volatile(__VA_ARGS__)
#else
#define CA_DEVICE_ASM(...) (void)0
#endif

template <int OFF>
__device__ __forceinline__ u32x2 lds_read_tr8(uint32_t a) {
  u32x2 r = {a, a};
  CA_DEVICE_ASM("ds_read_b64_tr_b8 %0, %1 offset:%2" : "=v"(r) : "v"(a), "n"(OFF));
  return r;
}
template <int OFF>
__device__ __forceinline__ u32x2 lds_read_tr16(uint32_t a) {
  u32x2 r = {a, a};
  CA_DEVICE_ASM("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(a), "n"(OFF));
  return r;
}
template <int OFF>
__device__ __forceinline__ uint32_t lds_read_b32(uint32_t a) {
  uint32_t r = a;
  CA_DEVICE_ASM("ds_read_b32 %0, %1 offset:%2" : "=v"(r) : "v"(a), "n"(OFF));
  return r;
}
template <int OFF>
__device__ __forceinline__ u32x2 lds_read_b64(uint32_t a) {
  u32x2 r = {a, a};
  CA_DEVICE_ASM("ds_read_b64 %0, %1 offset:%2" : "=v"(r) : "v"(a), "n"(OFF));
  return r;
}
template <int OFF>
__device__ __forceinline__ u32x4 lds_read_b128(uint32_t a) {
  u32x4 r = {a, a, a, a};
  CA_DEVICE_ASM("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(a), "n"(OFF));
  return r;
}
// LDS write by hand, for LDS the compiler would otherwise not write before
// every LDS DMA in flight has landed (it cannot tell the regions apart).
template <int OFF>
__device__ __forceinline__ void lds_write_b64(uint32_t a, u32x2 v) {
  CA_DEVICE_ASM("ds_write_b64 %0, %1 offset:%2" ::"v"(a), "v"(v), "n"(OFF));
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  CA_DEVICE_ASM("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_lgkm() {
  CA_DEVICE_ASM("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkm0() { wait_lgkm<0>(); }
// wait_lgkm<n> for an n that is a constant once the caller's loop is unrolled
// (the switch folds away); lgkmcnt holds at most 15.
__device__ __forceinline__ void wait_lgkm_n(int n) {
  switch (n) {
    case 0: wait_lgkm<0>(); break;
    case 1: wait_lgkm<1>(); break;
    case 2: wait_lgkm<2>(); break;
    case 3: wait_lgkm<3>(); break;
    case 4: wait_lgkm<4>(); break;
    case 5: wait_lgkm<5>(); break;
    case 6: wait_lgkm<6>(); break;
    case 7: wait_lgkm<7>(); break;
    case 8: wait_lgkm<8>(); break;
    case 9: wait_lgkm<9>(); break;
    case 10: wait_lgkm<10>(); break;
    case 11: wait_lgkm<11>(); break;
    case 12: wait_lgkm<12>(); break;
    case 13: wait_lgkm<13>(); break;
    case 14: wait_lgkm<14>(); break;
    default: wait_lgkm<15>(); break;
  }
}

// 16 bytes per lane from `src` into LDS at `dst` + 16 * lane (dst is
// wave-uniform: it is passed in M0). AUX is the cache policy: 0 = default
// (data re-read by other workgroups stays in L2), 2 = nt (streamed once).
template <int AUX>
__device__ __forceinline__ void dma16(const void* src, CA_LDS void* dst) {
  __builtin_amdgcn_global_load_lds(src, dst, 16, 0, AUX);
}

// Buffer-resource form: 16 bytes per lane from rsrc at byte offset `voffset`
// into LDS at `dst` + 16 * lane. A lane whose offset is at or past the
// resource's size reads zeros without a memory access, so a tile that runs
// past the end of a slice needs no clamping. The whole offset goes in the
// per-lane operand, which the range check covers (the scalar offset operand
// is left 0: whether the check includes it is not something to rely on).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  // word 3 = 0x00020000: 32-bit data format, as raw dword loads on gfx9 need
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t rsrc, CA_LDS void* dst,
                                          uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst, 16, (int)voffset, 0, 0, 0);
}
// 4 bytes per lane (LDS at `dst` + 4 * lane), same range check.
__device__ __forceinline__ void dma4_buf(__amdgpu_buffer_rsrc_t rsrc, CA_LDS void* dst,
                                         uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst, 4, (int)voffset, 0, 0, 0);
}

// Resource over bytes [off, size) of `base` (none when off >= size): a tile
// walk moves the resource rather than the per-lane offsets, which costs
// scalar instructions only. The arguments are wave-uniform; readfirstlane
// on the inputs says so to the compiler, which then computes the clamped
// size with scalar instructions (clamping after the readfirstlane instead
// costs a saturating vector subtract, a readfirstlane and its wait states
// per load) and does not wrap the load in a loop over distinct resources.
// Sizes are below 2^31 bytes (one (b, head) slice).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_at(const void* base, uint32_t off,
                                                               uint32_t size) {
  const int o = __builtin_amdgcn_readfirstlane((int)off);
  const int s = __builtin_amdgcn_readfirstlane((int)size);
  const int left = s > o ? s - o : 0;
  return make_rsrc((const char*)base + o, (uint32_t)left);
}

// Orders later uses of `x` after the preceding wait (the asm "rewrites" it).
template <typename T>
__device__ __forceinline__ void after_wait(T& x) {
  CA_DEVICE_ASM("" : "+v"(x));
}

}  // namespace ca
