// Prefill for 16-bit head dim 128 (bf16 or fp16): one wave per SIMD, 64
// query rows per wave, the key walk as hand-scheduled gfx950 assembly.
//
// Computes O = softmax(Q K^T * scale [+ causal mask]) V per (batch, q-head),
// the contract of dispatch_flash_attention_v2 / _v3_hopper / fused_gqa in the
// reference (kernels_api.h:29-33,52-56,78-83; math flash_attention_v2_kernel.cuh:
// 82-83 causal tile bound, 179-229 online softmax, 223 l == 0 -> 0), for
// softmax scales >= 0 (prefill.hip serves negative scales and the other head
// dims and element types).
//
// Work decomposition: one query tile = 256 rows of one (b, h), taken by the
// 4 waves of a workgroup (64 rows each); causal launches pair query tiles n-1-p
// and p of a head; with more items than CUs one workgroup per CU takes items
// g, g + grid, ... (prefill_work, xcd_remap in common.h, restated in the
// kernel body with magic-number divisions). K and V tiles of 64 keys travel
// HBM -> LDS by buffer loads into two rings of 4 tiles (K tile t is read by
// QK in iteration t - 1, V tile t by PV in iteration t + 1, so the rings
// release their slots at different times), every wave loading a quarter of
// each tile. The walk's code has a copy per iteration index mod 4, so every
// ring slot is an instruction offset on LDS addresses fixed for the kernel.
//
// Per wave, iteration i of the walk issues 64 v_mfma_f32_32x32x16_bf16 (_f16):
//   PV(i - 1): O^T[128 d x 64 q] += V^T P^T   (A = V^T via ds_read_b64_tr_b16,
//              B = P^T in VGPRs, O^T accumulators in AGPRs)
//   QK(i + 1): S^T[64 keys x 64 q] = K Q^T    (A = K from LDS, B = Q in AGPRs,
//              S^T accumulators in VGPRs, two buffers by tile parity)
// and between them the softmax of tile i: P = 2^(S c - m) against the
// running max m as it stands (a tile is redone with its own max, O and l
// rescaled, when a lane's tile sum passes 2^48 (fp16: 2^15, so no weight
// overflows its type) or is not finite), packed to bf16 / fp16 straight into
// the PV B operand, row sums as fp32 adds of the unrounded weights. Each K or V^T fragment read from LDS feeds two MFMAs (the wave's
// two 32-query blocks). The register assignment and the instruction order
// are fixed by gen_prefill_w64.py, which writes the body and checks its
// hazards and memory-counter waits.
//
// Lane layouts (32x32x16 MFMA, lane l = 32 h + l32):
//   A operand: row l32, k = 8 h + [0, 8); B: column l32, k = 8 h + [0, 8);
//   accumulator register r: row 8 (r / 4) + 4 h + r % 4, column l32.
//   The K fragment of lane l reads key row rho(l32) (bits 2 and 3 swapped),
//   so accumulator register r of lane half h holds key 16 (r / 8) + 8 h + r % 8
//   of its 32-key block: registers 8j..8j+7 are the PV B operand of k-step
//   2 mb + j as they stand (prefill.hip uses the same permutation).
#include <stddef.h>

#include "common.h"
#include "launch.h"
#include "prefill_w64_body.inc"

namespace ca {

// Kernel arguments; the body loads them from the kernarg segment at these
// offsets (gen_prefill_w64.py, KARG).
struct PfW64Args {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  int S, n_qt, n_work, paired, q_shift;
  float scale_log2;
  int n_bh, n_full, half, hq, hkv;
  // x / d = (x * m) >> sh for 0 <= x < 2^31 (magic division), per divisor
  uint32_t m_nqt, sh_nqt, m_half, sh_half, m_hq, sh_hq, m_ratio, sh_ratio;
  int xcd_q, xcd_r, pad;
};
static_assert(sizeof(PfW64Args) == 128, "kernel argument block");
static_assert(offsetof(PfW64Args, S) == 40 && offsetof(PfW64Args, scale_log2) == 60 &&
                  offsetof(PfW64Args, n_bh) == 64 && offsetof(PfW64Args, m_nqt) == 84 &&
                  offsetof(PfW64Args, xcd_q) == 116,
              "offsets the kernel body loads");

constexpr int kW64Threads = 256;  // 4 waves, one per SIMD (512 registers each)

template <bool CAUSAL, bool F16>
__global__ __launch_bounds__(kW64Threads, 1) void prefill_w64_kernel(PfW64Args args) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[160 * 1024];
  const int tid = threadIdx.x;
  const int lane = tid & 63, l32 = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  auto swz = [](int r) { return ((r & 3) << 2) | ((r >> 2) & 3); };
  // K fragment: key row krow (rho(l32)), logical chunk 2 ks + h of its 256 bytes
  const int krow = (l32 & 0x13) | ((l32 & 4) << 1) | ((l32 & 8) >> 1);
  const int fk = swz(krow);
  const int kofs = krow * 256 + 32 * (fk >> 1) + 16 * (h ^ (fk & 1));
  // V^T fragment: tr16 source row tr_row (+4 for the second read), chunk c0
  const int g16 = lane >> 4, s16 = lane & 15;
  const int tr_row = 8 * (g16 >> 1) + (s16 >> 2);
  const int c0 = 2 * (g16 & 1) + ((s16 & 3) >> 1);
  const int fv = swz(tr_row), fv2 = fv + 1;  // swz(tr_row + 4) (tr_row % 8 < 4)
  const int vofs1 = tr_row * 256 + 64 * (fv >> 2) + 16 * (c0 ^ (fv & 3)) + 8 * (s16 & 1);
  const int vofs2 = (tr_row + 4) * 256 + 64 * (fv2 >> 2) + 16 * (c0 ^ (fv2 & 3)) + 8 * (s16 & 1);
  // HBM -> LDS: load j of this wave covers tile rows 16 wave + 4 j + lane / 16;
  // the lane fetches the chunk that belongs at position lane % 16. The load's
  // instruction offset (1 KB j) adds to both addresses, so loff[j] leaves out
  // the 4 j rows.
  int loff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 16 * wave + 4 * j + (lane >> 4);
    loff[j] = row * 256 + 16 * ((lane & 15) ^ swz(row)) - 1024 * j;
  }
  const int qlane = l32 * 256 + 16 * h;          // Q row l32, bytes 16 h of each 32
  const int dl = l32 - 8 * h;                    // causal mask: key > query
  const int h8 = 8 * h;                          // key >= S mask
  const int wbase = 128 * l32 + 8 * h;           // output staging write: row l32
  const int wx = 16 * (l32 & 7);                 // chunk c at c ^ (row % 8)
  const int rdl = 128 * (lane >> 3) + 16 * ((lane & 7) ^ ((lane >> 3) & 7));  // staging read
  const int stl = (lane >> 3) * 256 + 16 * (lane & 7);                        // global row part
  const unsigned lsel = h ? 0x80000000u : (unsigned)(l32 * 4);                // LSE: lanes h = 0
  const unsigned lds_base = (unsigned)(uintptr_t)(const CA_LDS void*)lds;
#if __HIP_DEVICE_COMPILE__
#define CA_PFW64_OPERANDS                                                                         \
  [ka] "s"(__builtin_amdgcn_kernarg_segment_ptr()), [wg] "s"((int)blockIdx.x),                    \
      [ng] "s"((int)gridDim.x), [wv] "s"(wave), [lb] "s"(lds_base), [kofs] "v"(kofs),             \
      [vofs1] "v"(vofs1), [vofs2] "v"(vofs2), [loff0] "v"(loff[0]), [loff1] "v"(loff[1]),         \
      [loff2] "v"(loff[2]), [loff3] "v"(loff[3]), [qlane] "v"(qlane), [dl] "v"(dl), [h8] "v"(h8), \
      [wbase] "v"(wbase), [wx] "v"(wx), [rdl] "v"(rdl), [stl] "v"(stl), [lsel] "v"(lsel)
  if constexpr (CAUSAL && F16) {
    asm volatile(CA_PFW64_F16_BODY_CAUSAL ::CA_PFW64_OPERANDS : CA_PFW64_CLOBBERS);
  } else if constexpr (F16) {
    asm volatile(CA_PFW64_F16_BODY_FULL ::CA_PFW64_OPERANDS : CA_PFW64_CLOBBERS);
  } else if constexpr (CAUSAL) {
    asm volatile(CA_PFW64_BODY_CAUSAL ::CA_PFW64_OPERANDS : CA_PFW64_CLOBBERS);
  } else {
    asm volatile(CA_PFW64_BODY_FULL ::CA_PFW64_OPERANDS : CA_PFW64_CLOBBERS);
  }
#undef CA_PFW64_OPERANDS
#else
  (void)args;
  (void)kofs, (void)vofs1, (void)vofs2, (void)loff, (void)qlane, (void)dl, (void)h8, (void)wbase;
  (void)wx, (void)rdl, (void)stl, (void)lsel, (void)lds_base;
#endif
}

// x / d == (x * m) >> sh for 0 <= x < 2^31: s = ceil(log2 d), m = ceil(2^(31+s) / d)
// (m < 2^32 since d > 2^(s-1); the error term x (m d - 2^(31+s)) / (d 2^(31+s))
// stays below 1/d because m d - 2^(31+s) < d <= 2^s).
void magic_div(uint32_t d, uint32_t* m, uint32_t* sh) {
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  const unsigned long long num = 1ull << (31 + s);
  *m = (uint32_t)((num + d - 1) / d);
  *sh = 31 + s;
}

bool prefill_w64_supported(int D, int S, float scale, bool rope) {
  const float sl2 = scale * kLog2e;
  // S * 256 bytes per head must fit the 31-bit buffer offsets
  return D == 128 && !rope && sl2 >= 0.f && sl2 <= 3.0e38f && S > 0 && S < (1 << 22);
}

hipError_t w64_geometry(int B, int Hq, int S, bool causal, PfW64Geom* g) {
  constexpr int kRows = 256, kBN = 64;
  *g = PfW64Geom{};
  const int n_qt = (S + kRows - 1) / kRows;
  // padding rows of a ragged S go before row 0, in whole key tiles, so every
  // wave's causal diagonal is its last key tile
  g->q_shift = (n_qt * kRows - S) / kBN * kBN;
  const long long n_work = prefill_grid(B, Hq, n_qt, causal, 1, &g->paired);
  if (n_work == 0) return hipSuccess;
  if (n_work > 0x7fffffffLL || (long long)B * Hq > 0x7fffffffLL) return hipErrorInvalidValue;
  const long long slots = device_cus() / 8 * 8;
  g->grid = ((!causal || g->paired) && slots > 0 && n_work > slots) ? slots : n_work;
  g->n_qt = n_qt;
  g->n_work = (int)n_work;
  g->n_bh = B * Hq;
  g->half = n_qt >> 1;
  g->n_full = g->n_bh * g->half;
  magic_div((uint32_t)n_qt, &g->m_nqt, &g->sh_nqt);
  magic_div((uint32_t)(g->half > 0 ? g->half : 1), &g->m_half, &g->sh_half);
  g->xcd_q = (int)(n_work / 8);
  g->xcd_r = (int)(n_work % 8);
  return hipSuccess;
}

hipError_t launch_prefill_w64(bool f16, const void* q, const void* k, const void* v, void* o, float* lse, int B,
                              int Hq, int Hkv, int S, float scale, bool causal, hipStream_t stream) {
  PfW64Geom g;
  const hipError_t ge = w64_geometry(B, Hq, S, causal, &g);
  if (ge != hipSuccess || g.grid == 0) return ge;
  const long long grid = g.grid;
  PfW64Args a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = lse;
  a.S = S;
  a.n_qt = g.n_qt;
  a.n_work = g.n_work;
  a.paired = g.paired;
  a.q_shift = g.q_shift;
  a.scale_log2 = scale * kLog2e;
  a.n_bh = g.n_bh;
  a.half = g.half;
  a.n_full = g.n_full;
  a.hq = Hq;
  a.hkv = Hkv;
  a.m_nqt = g.m_nqt;
  a.sh_nqt = g.sh_nqt;
  a.m_half = g.m_half;
  a.sh_half = g.sh_half;
  magic_div((uint32_t)Hq, &a.m_hq, &a.sh_hq);
  magic_div((uint32_t)(Hq / Hkv), &a.m_ratio, &a.sh_ratio);
  a.xcd_q = g.xcd_q;
  a.xcd_r = g.xcd_r;
  const dim3 g3((unsigned)grid), b3(kW64Threads);
  if (causal && f16) {
    hipLaunchKernelGGL((prefill_w64_kernel<true, true>), g3, b3, 0, stream, a);
  } else if (f16) {
    hipLaunchKernelGGL((prefill_w64_kernel<false, true>), g3, b3, 0, stream, a);
  } else if (causal) {
    hipLaunchKernelGGL((prefill_w64_kernel<true, false>), g3, b3, 0, stream, a);
  } else {
    hipLaunchKernelGGL((prefill_w64_kernel<false, false>), g3, b3, 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace ca
