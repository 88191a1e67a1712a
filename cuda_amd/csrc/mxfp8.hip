// MXFP8 attention for gfx950: q, k, v are OCP e4m3 codes [B, H, S, D] with one
// e8m0 scale per 32 consecutive elements along D ([B, H, S, D/32]), given as
// e8m0 bytes or as float32 powers of two.
//
// The reference declares the entry point (dispatch_fused_microscaled_attention,
// kernels_api.h:103-108, float scales; README.md:29-31,80-81) but ships no
// kernel; the semantics here are attention over the dequantised tensors
// x = code * scale, fp32 accumulation, 16-bit output.
//
// Two launches:
//   mx_prepare_kernel: V dequantised exactly into bf16 (e4m3 * 2^e is a bf16
//     value) in the caller's workspace, once per launch rather than once per
//     query tile; with float scales it also converts q's and k's scales to
//     e8m0 bytes there. A float scale that is not a power of two in
//     [2^-127, 2^127] becomes the e8m0 NaN (0xFF), so the outputs it reaches
//     are not meaningful (NaN, or 0 for a row whose logits are all NaN); the
//     call stays asynchronous, and check_mx_scales (a separate, synchronous
//     entry) reports such scales;
//   the 64-row prefill kernel with MX operands (prefill_w64_mx.hip): QK on
//   v_mfma_scale_f32_32x32x64_f8f6f4 with the e8m0 bytes as per-lane scales,
//   softmax and PV (bf16 MFMA on the dequantised V) as in the bf16 kernel.
//   Limits: a finite softmax scale (a negative one is applied to -Q), S below
//   2^22 and B * H * S below 2^30 rows; otherwise the call fails before
//   launching anything.
#include <algorithm>

#include "common.h"
#include "launch.h"

namespace ca {

// e8m0 byte of a float32 scale: 2^k -> k + 127; anything that is not a power
// of two with k in [-127, 127] (2^-127 is the fp32 subnormal 0x00400000)
// gives 0xFF (NaN) and false.
__device__ __forceinline__ bool float_to_e8m0(float x, uint32_t* e) {
  const uint32_t u = __float_as_uint(x);
  if (u == 0x00400000u) {
    *e = 0;
    return true;
  }
  const uint32_t be = u >> 23;
  const bool ok = (u & 0x807fffffu) == 0 && be >= 1 && be <= 254;
  *e = ok ? be : 0xffu;
  return ok;
}

__device__ __forceinline__ float e8m0_to_float(uint32_t e) {
  // 2^(e-127); e = 0 is the fp32 subnormal 2^-127, e = 255 is NaN
  if (e == 0) return __uint_as_float(0x00400000u);
  if (e == 255) return __uint_as_float(0x7fc00000u);
  return __uint_as_float(e << 23);
}

// One wave per kMxPrepRows rows of V (kMxPrepRows x 128 codes): lane l
// converts codes 8l .. 8l + 7 of each 512-code quarter-block (4 rows), so every
// load instruction reads one contiguous 512 B and every store instruction
// writes one contiguous 1 KB of bf16; all of the wave's loads are issued
// before its first conversion, so a wave keeps kMxPrepRows x 128 bytes in
// flight. C5's 50 MB (kernel averages, one box): 8 rows per wave 11.8 µs,
// 16 rows 11.2 µs, 32 rows 14.8 µs (too few waves); 16 codes per lane with
// two 16-byte stores 32 bytes apart ran at ~3.4 TB/s. With float scales (F32SC)
// lane l also converts one q or k scale per 8 rows (row l / 8, block l % 4;
// q when (l / 4) % 2 == 0) into e8m0.
constexpr int kMxPrepRows = 16;
template <bool F32SC>
__global__ __launch_bounds__(256) void mx_prepare_kernel(
    const uint8_t* __restrict__ V, const void* __restrict__ VS, const void* __restrict__ QSf,
    const void* __restrict__ KSf, uint16_t* __restrict__ Vb, uint8_t* __restrict__ QSb,
    uint8_t* __restrict__ KSb, long long n_rows) {
  constexpr int D = 128, NB = D / 32, NH = kMxPrepRows / 4;
  const int lane = threadIdx.x & 63;
  const long long row0 = (((long long)blockIdx.x * 256 + threadIdx.x) >> 6) * kMxPrepRows;
  if (row0 >= n_rows) return;
  if (F32SC) {
#pragma unroll
    for (int g = 0; g < kMxPrepRows / 8; ++g) {
      const long long r = row0 + 8 * g + (lane >> 3);
      const int blk = lane & 3;
      if (r < n_rows) {
        const bool isq = ((lane >> 2) & 1) == 0;
        uint32_t e;
        float_to_e8m0(((const float*)(isq ? QSf : KSf))[r * NB + blk], &e);
        (isq ? QSb : KSb)[r * NB + blk] = (uint8_t)e;
      }
    }
  }
  const int blk = (lane & 15) >> 2;  // MX block of the lane's 8 codes
  u32x2 cc[NH];
  float sc[NH];
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const long long r = row0 + 4 * h + (lane >> 4);
    if (r >= n_rows) continue;
    cc[h] = *(const u32x2*)(V + row0 * D + 512 * h + 8 * lane);
    if (F32SC) {
      uint32_t e;
      float_to_e8m0(((const float*)VS)[r * NB + blk], &e);
      sc[h] = e8m0_to_float(e);
    } else {
      sc[h] = e8m0_to_float(((const uint8_t*)VS)[r * NB + blk]);
    }
  }
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const long long r = row0 + 4 * h + (lane >> 4);
    if (r >= n_rows) continue;
    u32x4 w;
    w[0] = __builtin_bit_cast(uint32_t, e4m3x2_to_bf16_scaled<false>(cc[h][0], sc[h]));
    w[1] = __builtin_bit_cast(uint32_t, e4m3x2_to_bf16_scaled<true>(cc[h][0], sc[h]));
    w[2] = __builtin_bit_cast(uint32_t, e4m3x2_to_bf16_scaled<false>(cc[h][1], sc[h]));
    w[3] = __builtin_bit_cast(uint32_t, e4m3x2_to_bf16_scaled<true>(cc[h][1], sc[h]));
    *(u32x4*)(Vb + row0 * D + 512 * h + 8 * lane) = w;
  }
}

// Raises *bad for any of the n float scales that is not a power of two in
// [2^-127, 2^127] (every writer stores the same value).
__global__ __launch_bounds__(256) void mx_check_scales_kernel(const float* __restrict__ s, long long n,
                                                              uint32_t* __restrict__ bad) {
  bool ok = true;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {
    uint32_t e;
    ok &= float_to_e8m0(s[i], &e);
  }
  if (!ok) *bad = 1u;
}

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Workspace: the bf16 V ([B, H, S, D]); with float scales also q's and k's
// e8m0 bytes ([B, H, S, D/32] each).
size_t mx_workspace_bytes(int scale_kind, int B, int H, int S, int D) {
  const size_t rows = (size_t)B * H * S;
  size_t n = align256(rows * D * 2);
  if (scale_kind == 1) n += 2 * align256(rows * (D / 32));
  return n;
}

// Synchronous check of three float scale arrays of n entries each: waits for
// `stream`, then sets *bad if any scale is not a power of two in
// [2^-127, 2^127]. Allocates (and frees) a 4-byte flag.
hipError_t check_mx_scales(const float* qs, const float* ks, const float* vs, long long n, bool* bad,
                           hipStream_t stream) {
  *bad = false;
  if (n <= 0) return hipSuccess;
  uint32_t* flag = nullptr;
  hipError_t e = hipMalloc((void**)&flag, sizeof(uint32_t));
  if (e != hipSuccess) return e;
  uint32_t h = 0;
  e = hipMemsetAsync(flag, 0, sizeof(uint32_t), stream);
  const long long blocks = std::min<long long>((n + 255) / 256, 4096);
  for (const float* s : {qs, ks, vs}) {
    if (e != hipSuccess) break;
    hipLaunchKernelGGL(mx_check_scales_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, s, n, flag);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpyAsync(&h, flag, sizeof(h), hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  const hipError_t ef = hipFree(flag);
  if (e == hipSuccess) e = ef;
  *bad = e == hipSuccess && h != 0;
  return e;
}

hipError_t launch_mxfp8(int out_dtype, int scale_kind, const uint8_t* q, const void* qs,
                        const uint8_t* k, const void* ks, const uint8_t* v, const void* vs, void* o,
                        int B, int H, int S, int D, float scale, bool causal, void* ws,
                        size_t ws_bytes, hipStream_t stream) {
  if (D != 128 || (out_dtype != kDtypeBF16 && out_dtype != kDtypeF16)) return hipErrorInvalidValue;
  const long long rows = (long long)B * H * S;
  if (rows == 0) return hipSuccess;
  // the attention kernel's limits (checked before the prepare launch)
  if (!prefill_w64_supported(128, S, scale < 0.f ? -scale : scale, false) || rows >= (1LL << 30))
    return hipErrorInvalidValue;
  if (ws_bytes < mx_workspace_bytes(scale_kind, B, H, S, D)) return hipErrorInvalidValue;
  unsigned char* w = (unsigned char*)ws;
  uint16_t* vb = (uint16_t*)w;
  w += align256((size_t)rows * D * 2);
  const uint8_t* qs8 = (const uint8_t*)qs;
  const uint8_t* ks8 = (const uint8_t*)ks;
  const long long blocks = (rows + 4 * kMxPrepRows - 1) / (4 * kMxPrepRows);  // 4 waves per block
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  if (scale_kind == 1) {
    uint8_t* qsb = w;
    uint8_t* ksb = w + align256((size_t)rows * (D / 32));
    hipLaunchKernelGGL(mx_prepare_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, v, vs,
                       qs, ks, vb, qsb, ksb, rows);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    qs8 = qsb;
    ks8 = ksb;
  } else {
    hipLaunchKernelGGL(mx_prepare_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, v, vs,
                       nullptr, nullptr, vb, nullptr, nullptr, rows);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return launch_prefill_w64_mx(out_dtype == kDtypeF16, q, qs8, k, ks8, vb, o, B, H, S, scale, causal, stream);
}

}  // namespace ca
