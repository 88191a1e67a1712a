// Paged KV-cache append for gfx950: the step before paged decode.
//
// New tokens key/value [N, Hkv, T, D] (16-bit) are written into the paged
// cache layout of the reference, cache[num_blocks, Hkv, D, 16] with the page
// axis innermost (tests/_utils.py:105-133; walk paged_attention_kernel.cuh:
// 61-76,86): token at position t of sequence n goes to page
// block_tables[n][t / 16], slot t % 16. Sequence n appends its first
// new_lens[n] tokens at positions context_lens[n] onwards. The reference has
// no kernel for this step; the FP8 form follows its quantisation recipe
// (tests/test_kernels_misc.py:52-55: scale = max(amax / 448, 1e-8), codes =
// e4m3 round-to-nearest-even of x / scale), per (page, kv head) as the
// [num_blocks, Hkv] scale form of the FP8 decode binding
// (fused_softmax_binding.cpp:640,671) expects.
//
// One wave per (sequence, kv head, touched page); lane l owns the page rows
// d = l + 64 i (a row is the 16 slots of one head dimension: 32 bytes for a
// 16-bit cache, 16 for FP8), so the token reads of a slot are coalesced
// across lanes and each row is read and written once.
//   16-bit cache: the new slots of each row are replaced;
//   FP8, per-head scales [Hkv]: new slots get e4m3(x / s[h]) (saturated);
//   FP8, per-page scales [num_blocks, Hkv]: the page is quantised again over
//     its valid slots (old slots decoded with the page's old scale, new slots
//     as given; amax over the whole page by a wave reduction); slots past the
//     new end get code 0.
// Positions past the block table and block ids outside [0, num_blocks) are
// skipped, never clamped (a write to a clamped block would corrupt another
// sequence's page).
#include "common.h"
#include "launch.h"

namespace ca {
namespace {

constexpr int kPage = 16;
constexpr float kE4m3Max = 448.f;

// float -> e4m3 (OCP) code, round to nearest even, saturated to +-448.
__device__ __forceinline__ uint32_t e4m3_code(float x) {
  x = __builtin_fminf(__builtin_fmaxf(x, -kE4m3Max), kE4m3Max);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x, 0.f, 0, false) & 0xffu;
}
__device__ __forceinline__ float e4m3_value(uint32_t code) {
  return __builtin_amdgcn_cvt_f32_fp8((int)code, 0);
}

__device__ __forceinline__ float wave_max_f(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = __builtin_fmaxf(x, __shfl_xor(x, m, 64));
  return x;
}

// KIND: 0 = 16-bit cache, 1 = FP8 with per-head scales, 2 = FP8 with
// per-(page, head) scales.
template <typename Tr, int D, int KIND>
__global__ __launch_bounds__(64) void kv_append_kernel(
    const uint16_t* __restrict__ key, const uint16_t* __restrict__ value, void* __restrict__ kc,
    void* __restrict__ vc, float* __restrict__ ks, float* __restrict__ vs,
    const int32_t* __restrict__ block_tables, const int32_t* __restrict__ context_lens,
    const int32_t* __restrict__ new_lens, int Hkv, int T, int max_blocks, int num_blocks,
    int max_touch) {
  constexpr int RPL = D / 64;  // rows per lane
  int w = blockIdx.x;
  const int j = w % max_touch;
  w /= max_touch;
  const int h = w % Hkv;
  const int n = w / Hkv;
  const int lo = max(0, context_lens[n]);
  const int nw = new_lens ? min(max(new_lens[n], 0), T) : T;
  const int hi = (int)min((long long)lo + nw, (long long)max_blocks * kPage);
  if (lo >= hi) return;
  const int page = lo / kPage + j;
  const int p0 = page * kPage;
  if (p0 >= hi) return;
  const int blk = block_tables[(size_t)n * max_blocks + page];
  if (blk < 0 || blk >= num_blocks) return;
  const int lane = threadIdx.x;

#pragma unroll
  for (int kv = 0; kv < 2; ++kv) {
    const uint16_t* src = (kv ? value : key) + (size_t)(n * Hkv + h) * T * D;
    if (KIND == 0) {
      uint16_t* cache = (uint16_t*)(kv ? vc : kc) + ((size_t)blk * Hkv + h) * D * kPage;
#pragma unroll
      for (int i = 0; i < RPL; ++i) {
        const int d = lane + 64 * i;
        u32x4* row = (u32x4*)(cache + (size_t)d * kPage);
        u32x4 r[2] = {row[0], row[1]};  // slot s: 16-bit half s % 2 of word s / 2
#pragma unroll
        for (int s = 0; s < kPage; ++s) {
          const int pos = p0 + s;
          if (pos >= lo && pos < hi) {
            const uint32_t x = src[(size_t)(pos - lo) * D + d];
            const uint32_t wd = r[s >> 3][(s >> 1) & 3];
            r[s >> 3][(s >> 1) & 3] = (s & 1) ? ((wd & 0xffffu) | (x << 16)) : ((wd & 0xffff0000u) | x);
          }
        }
        row[0] = r[0];
        row[1] = r[1];
      }
    } else {
      uint8_t* cache = (uint8_t*)(kv ? vc : kc) + ((size_t)blk * Hkv + h) * D * kPage;
      float* scales = kv ? vs : ks;
      if (KIND == 1) {
        const float s_h = scales[h];
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
          const int d = lane + 64 * i;
          u32x4* row = (u32x4*)(cache + (size_t)d * kPage);
          u32x4 r = row[0];  // slot s: byte s % 4 of word s / 4
#pragma unroll
          for (int s = 0; s < kPage; ++s) {
            const int pos = p0 + s;
            if (pos >= lo && pos < hi) {
              const uint32_t c = e4m3_code(Tr::to_float(src[(size_t)(pos - lo) * D + d]) / s_h);
              const int sh = 8 * (s & 3);
              r[s >> 2] = (r[s >> 2] & ~(0xffu << sh)) | (c << sh);
            }
          }
          row[0] = r;
        }
      } else {
        const float s_old = p0 < lo ? scales[(size_t)blk * Hkv + h] : 1.f;
        float x[RPL][kPage];
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
          const int d = lane + 64 * i;
          u32x4 r = u32x4{0, 0, 0, 0};
          if (p0 < lo) r = *(const u32x4*)(cache + (size_t)d * kPage);
#pragma unroll
          for (int s = 0; s < kPage; ++s) {
            const int pos = p0 + s;
            float val = 0.f;
            if (pos < lo) val = e4m3_value((r[s >> 2] >> (8 * (s & 3))) & 0xffu) * s_old;
            else if (pos < hi) val = Tr::to_float(src[(size_t)(pos - lo) * D + d]);
            x[i][s] = val;
            amax = __builtin_fmaxf(amax, __builtin_fabsf(val));
          }
        }
        amax = wave_max_f(amax);
        const float scale = __builtin_fmaxf(amax / kE4m3Max, 1e-8f);
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
          const int d = lane + 64 * i;
          u32x4 r = u32x4{0, 0, 0, 0};
#pragma unroll
          for (int s = 0; s < kPage; ++s)
            if (p0 + s < hi) r[s >> 2] |= e4m3_code(x[i][s] / scale) << (8 * (s & 3));
          *(u32x4*)(cache + (size_t)d * kPage) = r;
        }
        if (lane == 0) scales[(size_t)blk * Hkv + h] = scale;
      }
    }
  }
}

template <typename Tr, int D, int KIND>
hipError_t launch_t(const void* key, const void* value, void* kc, void* vc, float* ks, float* vs,
                    const int32_t* bt, const int32_t* lens, const int32_t* new_lens, int N,
                    int Hkv, int T, int max_blocks, int num_blocks, hipStream_t stream) {
  // a run of T tokens starting mid-page touches at most ceil(T / 16) + 1 pages
  const int max_touch = (T + kPage - 1) / kPage + 1;
  const long long grid = (long long)N * Hkv * max_touch;
  if (grid == 0) return hipSuccess;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((kv_append_kernel<Tr, D, KIND>), dim3((unsigned)grid), dim3(64), 0, stream,
                     (const uint16_t*)key, (const uint16_t*)value, kc, vc, ks, vs, bt, lens,
                     new_lens, Hkv, T, max_blocks, num_blocks, max_touch);
  return hipGetLastError();
}

template <typename Tr, int D>
hipError_t launch_d(int kind, const void* key, const void* value, void* kc, void* vc, float* ks,
                    float* vs, const int32_t* bt, const int32_t* lens, const int32_t* new_lens,
                    int N, int Hkv, int T, int max_blocks, int num_blocks, hipStream_t stream) {
  if (kind == 0)
    return launch_t<Tr, D, 0>(key, value, kc, vc, ks, vs, bt, lens, new_lens, N, Hkv, T,
                              max_blocks, num_blocks, stream);
  if (kind == 1)
    return launch_t<Tr, D, 1>(key, value, kc, vc, ks, vs, bt, lens, new_lens, N, Hkv, T,
                              max_blocks, num_blocks, stream);
  return launch_t<Tr, D, 2>(key, value, kc, vc, ks, vs, bt, lens, new_lens, N, Hkv, T,
                            max_blocks, num_blocks, stream);
}

}  // namespace

hipError_t launch_kv_append(int dtype, int kind, const void* key, const void* value, void* kc,
                            void* vc, float* k_scale, float* v_scale, const int32_t* block_tables,
                            const int32_t* context_lens, const int32_t* new_lens, int N, int Hkv,
                            int D, int T, int max_blocks, int num_blocks, hipStream_t stream) {
#define CA_APPEND_CASE(TR, DD)                                                                  \
  if (D == DD)                                                                                  \
    return launch_d<TR, DD>(kind, key, value, kc, vc, k_scale, v_scale, block_tables,           \
                            context_lens, new_lens, N, Hkv, T, max_blocks, num_blocks, stream);
  if (dtype == kDtypeBF16) {
    CA_APPEND_CASE(BF16, 64)
    CA_APPEND_CASE(BF16, 128)
  } else if (dtype == kDtypeF16) {
    CA_APPEND_CASE(F16, 64)
    CA_APPEND_CASE(F16, 128)
  }
#undef CA_APPEND_CASE
  return hipErrorInvalidValue;
}

}  // namespace ca
