// RoPE + prefill for gfx950: the fused_rope_flash_attention entry point.
//
// O = softmax(rope(Q) rope(K)^T * scale [+ causal]) V with the rotate-half
// RoPE of the reference (fused_rope_flash_attention_kernel.cuh:60-70,98-108;
// tests/_utils.py:75-94): for position s and dim c,
//   x'[c] = x[c] cos[s][c] + r[c] sin[s][c],  r = [-x[D/2:], x[:D/2]],
// with fp32 tables cos / sin [S, D].
//
// K is rotated once by rope_kernel into a caller-provided workspace (in the
// input dtype: that is the operand precision of the prefill kernels): every
// K row is read by many query tiles, so rotating it once is cheaper than
// rotating it in every tile that reads it (the pass is HBM-bound: k read and
// written once). Q is rotated by the 16-bit prefill kernels themselves as
// they load it into registers (rope_q in prefill.hip); for float32 q is
// rotated into the workspace as well. (The reference rotates both inside its
// attention loop.)
// One thread rotates 8 consecutive dims c .. c+7 of the first half together
// with their partners c+D/2 .. c+D/2+7.
#include "common.h"
#include "launch.h"

namespace ca {
namespace {

template <typename T>
struct Elem;
template <>
struct Elem<BF16> {
  static __device__ __forceinline__ float ld(const void* p, size_t i) {
    return BF16::to_float(((const uint16_t*)p)[i]);
  }
  static __device__ __forceinline__ void st(void* p, size_t i, float x) { BF16::store(p, i, x); }
};
template <>
struct Elem<F16> {
  static __device__ __forceinline__ float ld(const void* p, size_t i) {
    return F16::to_float(((const uint16_t*)p)[i]);
  }
  static __device__ __forceinline__ void st(void* p, size_t i, float x) { F16::store(p, i, x); }
};
template <>
struct Elem<F32> {
  static __device__ __forceinline__ float ld(const void* p, size_t i) { return ((const float*)p)[i]; }
  static __device__ __forceinline__ void st(void* p, size_t i, float x) { F32::store(p, i, x); }
};

// rows = heads * S rows of D elements; row r is at position r % S.
template <typename Tr, int D>
__global__ __launch_bounds__(256) void rope_kernel(const void* __restrict__ x, void* __restrict__ y,
                                                   const float* __restrict__ cos_tab,
                                                   const float* __restrict__ sin_tab,
                                                   long long rows, int S) {
  constexpr int H = D / 2;
  constexpr int L = H / 8;  // threads per row
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long row = t / L;
  if (row >= rows) return;
  const int c0 = 8 * (int)(t % L);
  const size_t base = (size_t)row * D;
  const size_t tab = (size_t)(row % S) * D;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int c = c0 + j;
    const float a = Elem<Tr>::ld(x, base + c);
    const float b = Elem<Tr>::ld(x, base + c + H);
    // x'[c] = a cos[c] - b sin[c];  x'[c + H] = b cos[c + H] + a sin[c + H]
    Elem<Tr>::st(y, base + c, a * cos_tab[tab + c] - b * sin_tab[tab + c]);
    Elem<Tr>::st(y, base + c + H, b * cos_tab[tab + c + H] + a * sin_tab[tab + c + H]);
  }
}

template <typename Tr, int D>
hipError_t rope_t(const void* x, void* y, const float* cos_tab, const float* sin_tab,
                  long long rows, int S, hipStream_t stream) {
  const long long threads = rows * (D / 16);
  const long long grid = (threads + 255) / 256;
  if (grid == 0) return hipSuccess;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((rope_kernel<Tr, D>), dim3((unsigned)grid), dim3(256), 0, stream, x, y,
                     cos_tab, sin_tab, rows, S);
  return hipGetLastError();
}

hipError_t rope(int dtype, int D, const void* x, void* y, const float* cos_tab,
                const float* sin_tab, long long rows, int S, hipStream_t stream) {
#define CA_ROPE_CASE(TR)                                                               \
  return D == 64 ? rope_t<TR, 64>(x, y, cos_tab, sin_tab, rows, S, stream)             \
                 : rope_t<TR, 128>(x, y, cos_tab, sin_tab, rows, S, stream);
  if (dtype == kDtypeBF16) { CA_ROPE_CASE(BF16) }
  if (dtype == kDtypeF16) { CA_ROPE_CASE(F16) }
  if (dtype == kDtypeF32) { CA_ROPE_CASE(F32) }
#undef CA_ROPE_CASE
  return hipErrorInvalidValue;
}

size_t elem_bytes(int dtype) { return dtype == kDtypeF32 ? 4 : 2; }

}  // namespace

// float32: rotated q, then k (256-byte aligned); 16-bit: rotated k only.
size_t rope_workspace_bytes(int dtype, int B, int Hq, int Hkv, int S, int D) {
  const size_t qb = (size_t)B * Hq * S * D * elem_bytes(dtype);
  const size_t kb = (size_t)B * Hkv * S * D * elem_bytes(dtype);
  return dtype == kDtypeF32 ? ((qb + 255) & ~(size_t)255) + kb : kb;
}

hipError_t launch_rope_prefill(int dtype, const void* q, const void* k, const void* v,
                               const float* cos_tab, const float* sin_tab, void* o, int B, int Hq,
                               int Hkv, int S, int D, float scale, bool causal, void* ws,
                               hipStream_t stream) {
  if (dtype != kDtypeF32) {
    hipError_t e = rope(dtype, D, k, ws, cos_tab, sin_tab, (long long)B * Hkv * S, S, stream);
    if (e != hipSuccess) return e;
    RopeQ rq;
    rq.cos = cos_tab;
    rq.sin = sin_tab;
    return launch_prefill(dtype, q, ws, v, o, nullptr, B, Hq, Hkv, S, D, scale, causal, stream, rq);
  }
  const size_t qb = (size_t)B * Hq * S * D * elem_bytes(dtype);
  void* qr = ws;
  void* kr = (char*)ws + ((qb + 255) & ~(size_t)255);
  hipError_t e = rope(dtype, D, q, qr, cos_tab, sin_tab, (long long)B * Hq * S, S, stream);
  if (e != hipSuccess) return e;
  e = rope(dtype, D, k, kr, cos_tab, sin_tab, (long long)B * Hkv * S, S, stream);
  if (e != hipSuccess) return e;
  return launch_prefill(dtype, qr, kr, v, o, nullptr, B, Hq, Hkv, S, D, scale, causal, stream);
}

}  // namespace ca
