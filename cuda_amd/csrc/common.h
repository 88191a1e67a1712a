// Shared device helpers for the gfx950 attention kernels.
//
// Everything here is written for CDNA4 (gfx950, wave64): MFMA operand vector
// types, 16-bit element traits (bf16 / fp16), LDS transpose reads, fp8 e4m3
// conversions and wave reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ca {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define CA_LDS __attribute__((address_space(3)))
// for lambdas inside kernels: they capture register arrays by reference
#define CA_INLINE __attribute__((always_inline))

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();

// ---------------------------------------------------------------------------
// 16-bit element traits: storage is raw uint16_t in HBM; MFMA operands are the
// clang vector types the gfx950 builtins take.
// ---------------------------------------------------------------------------
struct BF16 {
  using vec8 = bf16x8;
  using vec4 = bf16x4;
  using vec2 = bf16x2;
  static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  // 16x16x16: 4 elements of k per lane (k = 4 * (lane / 16) + 0..3)
  static __device__ __forceinline__ f32x4 mfma16k16(vec4 a, vec4 b, f32x4 c) {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                     __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ vec4 tr_read(const CA_LDS void* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((CA_LDS vec4*)p);
  }
  // round-to-nearest-even pack of two floats
  static __device__ __forceinline__ vec2 pack2(float a, float b) {
    vec2 r;
    r[0] = (__bf16)a;
    r[1] = (__bf16)b;
    return r;
  }
  static __device__ __forceinline__ float to_float(uint16_t x) {
    return __uint_as_float(((uint32_t)x) << 16);
  }
  // out[i] = x rounded to this type
  static __device__ __forceinline__ void store(void* out, size_t i, float x) {
    ((uint16_t*)out)[i] = __builtin_bit_cast(uint16_t, (__bf16)x);
  }
};

struct F16 {
  using vec8 = f16x8;
  using vec4 = f16x4;
  using vec2 = f16x2;
  static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16k16(vec4 a, vec4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ vec4 tr_read(const CA_LDS void* p) {
    typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));
    return __builtin_bit_cast(vec4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((CA_LDS fp16x4_t*)p));
  }
  static __device__ __forceinline__ vec2 pack2(float a, float b) {
    vec2 r;
    r[0] = (_Float16)a;
    r[1] = (_Float16)b;
    return r;
  }
  static __device__ __forceinline__ float to_float(uint16_t x) {
    _Float16 h = __builtin_bit_cast(_Float16, x);
    return (float)h;
  }
  static __device__ __forceinline__ void store(void* out, size_t i, float x) {
    ((uint16_t*)out)[i] = __builtin_bit_cast(uint16_t, (_Float16)x);
  }
};

// fp32 element type (only the output store is used by shared kernels).
struct F32 {
  static __device__ __forceinline__ void store(void* out, size_t i, float x) {
    ((float*)out)[i] = x;
  }
};

// ---------------------------------------------------------------------------
// Small helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Natural-log logsumexp of a softmax row from the online-softmax state: m is
// the running max of the scaled logits in log2 units, l the row sum of
// 2^(x - m); an empty row (l == 0) gives -inf. l >= 1 for a non-empty row
// (its largest term is 2^(max - m) >= 1), so the hardware log2 is accurate.
__device__ __forceinline__ float row_lse(float m, float l) {
  return l > 0.f ? (m + __builtin_amdgcn_logf(l)) * 0.6931471805599453f : kNegInf;
}

__device__ __forceinline__ float max3(float a, float b, float c) {
  return __builtin_fmaxf(a, __builtin_fmaxf(b, c));
}

// Reductions across lane pairs (lane, lane ^ 32) and (lane, lane ^ 16) with
// the gfx950 v_permlane32_swap / v_permlane16_swap: called with the same
// value as both operands, one of the two results is the lane's own value and
// the other its partner's, so max/sum of the pair needs no LDS traffic.
__device__ __forceinline__ float pair32_max(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair32_sum(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair16_max(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair16_sum(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ bool wave_any(bool p) { return __ballot(p) != 0ull; }

// LDS transpose read of 8 bytes (gfx950 ds_read_b64_tr_b8).
__device__ __forceinline__ i32x2 tr8_read(const CA_LDS void* p) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((CA_LDS i32x2*)p);
}

// fp8 e4m3 (OCP) x2 -> bf16 x2, exact (e4m3 values are bf16 values); HI
// selects bytes 2-3 instead of 0-1 of the dword.
template <bool HI>
__device__ __forceinline__ bf16x2 e4m3x2_to_bf16(uint32_t w) {
  return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI);
}
template <bool HI>
__device__ __forceinline__ f16x2 e4m3x2_to_f16(uint32_t w) {
  return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI);
}
// fp8 e4m3 x2 -> bf16 x2 multiplied by a power-of-two scale (exact unless the
// product leaves bf16's range).
template <bool HI>
__device__ __forceinline__ bf16x2 e4m3x2_to_bf16_scaled(uint32_t w, float s) {
  return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, s, HI);
}

template <typename V8, typename V4>
__device__ __forceinline__ V8 cat4(V4 lo, V4 hi) {
  V8 r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

// The lane index (0..63) recomputed where it is used, from v_mbcnt rather
// than the work-item id: the compiler can neither hoist it (volatile) nor keep
// the work-item id register live for it across a loop, which in the kernels
// at 256 VGPRs turned hoisted lane offsets into spills.
__device__ __forceinline__ int lane_here() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// Hardware XCD of workgroup `w`: consecutive workgroup ids are dealt
// round-robin over the 8 XCDs of an MI355X. Returns the logical work index so
// that each XCD walks one contiguous slice of [0, total).
__device__ __forceinline__ int xcd_remap(int w, int total) {
  constexpr int kXcd = 8;
  const int q = total / kXcd, r = total % kXcd;
  const int x = w % kXcd, i = w / kXcd;
  return (x < r) ? x * (q + 1) + i : r * (q + 1) + (x - r) * q + i;
}

// Query tiles of one prefill workgroup (work index after xcd_remap; n_bh =
// B * Hq heads, n_qt tiles per head). Unpaired: one tile; the work index runs
// over heads and, within a head, over its tiles longest causal walk first.
// Paired (causal launches, n_qt > 1): tiles n_qt-1-p and p of one head, whose
// causal key walks add up to the same length for every p, so all workgroups
// carry equal work and the grid ends without a tail of long workgroups; for
// an odd n_qt the middle tiles of heads 2m and 2m+1 make the last work items.
struct QTileWork {
  int bh0, qt0, bh1, qt1;  // qt1 < 0: no second tile
};
__device__ __forceinline__ QTileWork prefill_work(int work, int n_qt, int n_bh, int paired) {
  QTileWork w;
  w.bh1 = 0;
  w.qt1 = -1;
  if (!paired) {
    w.bh0 = work / n_qt;
    w.qt0 = n_qt - 1 - work % n_qt;
    return w;
  }
  const int half = n_qt >> 1;  // full pairs per head
  const int n_full = n_bh * half;
  if (work < n_full) {
    const int p = work % half;
    w.bh0 = w.bh1 = work / half;
    w.qt0 = n_qt - 1 - p;
    w.qt1 = p;
  } else {
    const int m = work - n_full;
    w.bh0 = 2 * m;
    w.qt0 = half;
    if (2 * m + 1 < n_bh) {
      w.bh1 = 2 * m + 1;
      w.qt1 = half;
    }
  }
  return w;
}

}  // namespace ca
