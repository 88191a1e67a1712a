// MXFP8 prefill for head dim 128 on the 64-row walk of prefill_w64.hip: one
// wave per SIMD, 64 query rows per wave, the key walk as hand-scheduled
// gfx950 assembly (gen_prefill_w64.py --mx).
//
// Computes O = softmax(Q K^T * scale [+ causal mask]) V per (batch, head) for
// dispatch_fused_microscaled_attention (kernels_api.h:103-108, which the
// reference declares without a kernel; semantics as mxfp8.hip states): Q and
// K are OCP e4m3 codes with one e8m0 scale byte per 32 elements along D
// ([rows][4]), V the exact bf16 dequantisation (mx_prepare_kernel), the
// output bf16 or fp16. A negative softmax scale c runs as |c| on -Q (the
// codes' sign bits flipped in registers at the start of each query tile).
//
// QK runs on v_mfma_scale_f32_32x32x64_f8f6f4 (16 passes): per 64-d k-step
// s2, lane half h supplies d = 64 s2 + 16 h + [0, 16) in bytes 0-15 and
// d = 64 s2 + 32 + 16 h + [0, 16) in bytes 16-31, with the scale of MX block
// 2 s2 + h, for K rows (the A operand, from LDS) and Q rows (B, AGPRs) alike.
// A lane keeps the scale bytes of its two key rows in one register (byte
// 2 mb + s2 for key block mb) and those of its two query rows in another
// (byte 2 nb + s2), and each MFMA picks its bytes with op_sel. PV, the
// softmax and the output are the bf16 walk's.
//
// LDS ring slot of a K tile (16 KB): 64 rows of 128 code bytes (chunk c of
// row r at c ^ swz128(r)), then at +8 KB the tile's 64 scale words. Each wave
// loads 16 code rows (2 x 1 KB) and all 64 scale words (every wave writes the
// same bytes, so each wave's own load covers its reads). All K and V^T
// fragments are read into AGPRs.
#include <stddef.h>

#include "common.h"
#include "launch.h"
#include "prefill_w64_mx_body.inc"

namespace ca {

// Kernel arguments; the body loads them from the kernarg segment at these
// offsets (the bf16 kernel's block, with the slots the MX kernel does not
// use for LSE and GQA carrying the scale pointers and the output type).
struct PfW64MxArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  const void* qs;
  int S, n_qt, n_work, paired, q_shift;
  float scale_log2;
  int n_bh, n_full, half, hq, unused0;
  uint32_t m_nqt, sh_nqt, m_half, sh_half;
  uint32_t flags, unused1, ks_lo, ks_hi;  // flags: bit 0 fp16 output, bit 1 negate Q
  int xcd_q, xcd_r, pad;
};
static_assert(sizeof(PfW64MxArgs) == 128, "kernel argument block");
static_assert(offsetof(PfW64MxArgs, qs) == 32 && offsetof(PfW64MxArgs, S) == 40 &&
                  offsetof(PfW64MxArgs, scale_log2) == 60 && offsetof(PfW64MxArgs, m_nqt) == 84 &&
                  offsetof(PfW64MxArgs, flags) == 100 && offsetof(PfW64MxArgs, ks_lo) == 108 &&
                  offsetof(PfW64MxArgs, xcd_q) == 116,
              "offsets the kernel body loads");

template <bool CAUSAL>
__global__ __launch_bounds__(256, 1) void prefill_w64_mx_kernel(PfW64MxArgs args) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[160 * 1024];
  const int tid = threadIdx.x;
  const int lane = tid & 63, l32 = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  auto swz = [](int r) { return ((r & 3) << 2) | ((r >> 2) & 3); };              // 256-byte rows (V)
  auto swz128 = [](int r) { return (((r >> 1) & 1) << 2) | ((r >> 2) & 3); };   // 128-byte rows (K codes)
  // K fragment: key row krow (rho(l32)), chunk pair 0: chunk h of its 128 bytes
  const int krow = (l32 & 0x13) | ((l32 & 4) << 1) | ((l32 & 8) >> 1);
  const int fk = swz128(krow);
  const int kofs = krow * 128 + 32 * (fk >> 1) + 16 * (h ^ (fk & 1));
  // V^T fragment (as the bf16 kernel)
  const int g16 = lane >> 4, s16 = lane & 15;
  const int tr_row = 8 * (g16 >> 1) + (s16 >> 2);
  const int c0 = 2 * (g16 & 1) + ((s16 & 3) >> 1);
  const int fv = swz(tr_row), fv2 = fv + 1;
  const int vofs1 = tr_row * 256 + 64 * (fv >> 2) + 16 * (c0 ^ (fv & 3)) + 8 * (s16 & 1);
  const int vofs2 = (tr_row + 4) * 256 + 64 * (fv2 >> 2) + 16 * (c0 ^ (fv2 & 3)) + 8 * (s16 & 1);
  // HBM -> LDS: V load j covers tile rows 16 wave + 4 j + lane / 16; K code
  // load j rows 16 wave + 8 j + lane / 8. The instruction offset (1 KB j)
  // adds to both addresses, so the offsets leave it out.
  int loff[4], kl[2];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 16 * wave + 4 * j + (lane >> 4);
    loff[j] = row * 256 + 16 * ((lane & 15) ^ swz(row)) - 1024 * j;
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int row = 16 * wave + 8 * j + (lane >> 3);
    kl[j] = row * 128 + 16 * ((lane & 7) ^ swz128(row)) - 1024 * j;
  }
  const int sl = 4 * lane;                                  // scale word of key row lane
  const unsigned lds_base = (unsigned)(uintptr_t)(const CA_LDS void*)lds;
  const unsigned ksr = lds_base + 4 * krow;                 // scale word of key row krow (+128: krow + 32)
  const unsigned psel = h ? 0x07050301u : 0x06040200u;      // bytes h, 2 + h of two words
  const int qlane = l32 * 128 + 16 * h;                     // Q row l32, bytes 16 h of each 32
  const int dl = l32 - 8 * h;                               // causal mask: key > query
  const int h8 = 8 * h;                                     // key >= S mask
  const int wbase = 128 * l32 + 8 * h;                      // output staging write: row l32
  const int wx = 16 * (l32 & 7);                            // chunk c at c ^ (row % 8)
  const int rdl = 128 * (lane >> 3) + 16 * ((lane & 7) ^ ((lane >> 3) & 7));  // staging read
  const int stl = (lane >> 3) * 256 + 16 * (lane & 7);                        // global row part
#if __HIP_DEVICE_COMPILE__
#define CA_PFW64MX_OPERANDS                                                                        \
  [ka] "s"(__builtin_amdgcn_kernarg_segment_ptr()), [wg] "s"((int)blockIdx.x),                    \
      [ng] "s"((int)gridDim.x), [wv] "s"(wave), [lb] "s"(lds_base), [kofs] "v"(kofs),             \
      [vofs1] "v"(vofs1), [vofs2] "v"(vofs2), [loff0] "v"(loff[0]), [loff1] "v"(loff[1]),         \
      [loff2] "v"(loff[2]), [loff3] "v"(loff[3]), [kl0] "v"(kl[0]), [kl1] "v"(kl[1]), [sl] "v"(sl), \
      [ksr] "v"(ksr), [psel] "v"(psel), [qlane] "v"(qlane), [dl] "v"(dl), [h8] "v"(h8),             \
      [wbase] "v"(wbase), [wx] "v"(wx), [rdl] "v"(rdl), [stl] "v"(stl)
  if constexpr (CAUSAL) {
    asm volatile(CA_PFW64MX_BODY_CAUSAL ::CA_PFW64MX_OPERANDS : CA_PFW64MX_CLOBBERS);
  } else {
    asm volatile(CA_PFW64MX_BODY_FULL ::CA_PFW64MX_OPERANDS : CA_PFW64MX_CLOBBERS);
  }
#undef CA_PFW64MX_OPERANDS
#else
  (void)args;
  (void)kofs, (void)vofs1, (void)vofs2, (void)loff, (void)kl, (void)sl, (void)ksr, (void)psel, (void)qlane;
  (void)dl, (void)h8, (void)wbase, (void)wx, (void)rdl, (void)stl, (void)lds_base;
#endif
}

hipError_t launch_prefill_w64_mx(bool out_f16, const uint8_t* q, const uint8_t* qs, const uint8_t* k,
                                 const uint8_t* ks, const uint16_t* v_bf16, void* o, int B, int H, int S,
                                 float scale, bool causal, hipStream_t stream) {
  const bool neg = scale < 0.f;
  if (neg) scale = -scale;
  // the Q scale words are read at 32-bit offsets from qs
  if (!prefill_w64_supported(128, S, scale, false) || (long long)B * H * S * 4 > 0xffffffffLL)
    return hipErrorInvalidValue;
  PfW64Geom g;
  const hipError_t ge = w64_geometry(B, H, S, causal, &g);
  if (ge != hipSuccess || g.grid == 0) return ge;
  PfW64MxArgs a{};
  a.q = q;
  a.k = k;
  a.v = v_bf16;
  a.o = o;
  a.qs = qs;
  a.S = S;
  a.n_qt = g.n_qt;
  a.n_work = g.n_work;
  a.paired = g.paired;
  a.q_shift = g.q_shift;
  a.scale_log2 = scale * kLog2e;
  a.n_bh = g.n_bh;
  a.n_full = g.n_full;
  a.half = g.half;
  a.hq = H;
  a.m_nqt = g.m_nqt;
  a.sh_nqt = g.sh_nqt;
  a.m_half = g.m_half;
  a.sh_half = g.sh_half;
  a.flags = (out_f16 ? 1u : 0u) | (neg ? 2u : 0u);
  a.ks_lo = (uint32_t)(uintptr_t)ks;
  a.ks_hi = (uint32_t)((uint64_t)(uintptr_t)ks >> 32);
  a.xcd_q = g.xcd_q;
  a.xcd_r = g.xcd_r;
  if (causal) {
    hipLaunchKernelGGL(prefill_w64_mx_kernel<true>, dim3((unsigned)g.grid), dim3(256), 0, stream, a);
  } else {
    hipLaunchKernelGGL(prefill_w64_mx_kernel<false>, dim3((unsigned)g.grid), dim3(256), 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace ca
