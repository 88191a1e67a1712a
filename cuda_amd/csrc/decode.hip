// Decode attention (q_len = 1) for gfx950: paged bf16/fp16 cache, paged FP8
// e4m3 cache with fp32 per-(page, kv-head) or per-head scales, and the
// contiguous [B, Hkv, S, D] cache of flash_decode. GQA throughout.
//
// Reference contracts: dispatch_paged_attention (kernels_api.h:35-41,
// paged_attention_kernel.cuh:20-182: block-table walk :61-76, element
// cache[p][h][d][t % 16] :86,127), dispatch_fp8_paged_attention
// (kernels_api.h:94-101, fp8_paged_attention_kernel.cuh:75-104,137: scale per
// head or per (block, head), logit scale folding, v-scale folding) and
// dispatch_async_flash_decode (kernels_api.h:58-62). The reference walks each
// (sequence, head) serially in one block; here contexts are split.
//
// Work decomposition (split-K, one wave per split)
//   a wave owns (sequence n, kv head, query-head chunk of <= 16, split) and
//   walks kPagesPerWave pages of 16 tokens, two pages per step, with the next
//   step's K and V already in flight in a second register set (the step loop
//   is unrolled by two so the sets swap roles without copies). Waves never
//   synchronise; a workgroup is just four independent waves.
//   The GQA group of query heads (Hq / Hkv <= 16 per chunk) shares every K/V
//   byte loaded, so each cache byte is read from HBM once per kv head.
// Per wave and step (16x16x32 MFMAs, query heads padded to 16):
//   S^T[16 tok x 16 heads] = K^T Q^T per page; a page is [D][16] with tokens
//   contiguous, so the K^T operand (8 consecutive d for one token) is read
//   from a wave-private LDS copy with ds_read_b64_tr_b16 / _tr_b8;
//   online softmax over tokens, rescaled only when the max grows by > 2^8;
//   O[16 heads x D] += P V^T over the step's 32 tokens; the V^T operand
//   (tokens contiguous for one d) is loaded from HBM in operand layout.
//   FP8: codes are converted exactly to the MFMA element type; the k scale of
//   a page multiplies that page's logits and the v scale is folded into P.
// A sequence that fits one split writes its output directly; otherwise each
// wave writes (o / l, log2-sum-exp) to the workspace and decode_merge_kernel
// combines the splits. (This describes the contiguous-cache kernel; the
// paged kernels below stream pages HBM -> LDS, and larger paged launches
// balance the pages over one wave per SIMD instead of splitting per
// sequence: decode_sk_kernel.)
#include <algorithm>
#include <atomic>
#include <climits>
#include <functional>
#include <mutex>

#include "common.h"
#include "launch.h"
#include "lds_dma.h"

namespace ca {

enum : int { kKindPaged16 = 0, kKindPagedFp8 = 1 };

template <typename Tr>
struct Fp8Conv;
template <>
struct Fp8Conv<BF16> {
  template <bool HI>
  static __device__ __forceinline__ BF16::vec2 cvt(uint32_t w) { return e4m3x2_to_bf16<HI>(w); }
};
template <>
struct Fp8Conv<F16> {
  template <bool HI>
  static __device__ __forceinline__ F16::vec2 cvt(uint32_t w) { return e4m3x2_to_f16<HI>(w); }
};

// 8 e4m3 codes (two dwords) -> 8 values of the MFMA element type; each
// conversion fills one dword, so the operand is assembled without shuffles
template <typename Tr>
__device__ __forceinline__ typename Tr::vec8 fp8x8_to(uint32_t lo, uint32_t hi) {
  const u32x4 r = {__builtin_bit_cast(uint32_t, Fp8Conv<Tr>::template cvt<false>(lo)),
                   __builtin_bit_cast(uint32_t, Fp8Conv<Tr>::template cvt<true>(lo)),
                   __builtin_bit_cast(uint32_t, Fp8Conv<Tr>::template cvt<false>(hi)),
                   __builtin_bit_cast(uint32_t, Fp8Conv<Tr>::template cvt<true>(hi))};
  return __builtin_bit_cast(typename Tr::vec8, r);
}

// Streaming loads: every cache byte is used once per launch, so they bypass
// the cache hierarchy's retention (non-temporal).
template <typename T>
__device__ __forceinline__ T ld_stream(const void* p) {
  return __builtin_nontemporal_load((const T*)p);
}

// Contiguous-cache decode (flash_decode): one wave per split of kPagesPerWave
// "pages" of 16 consecutive tokens of one (sequence, kv head, <= 16 q heads).
// K^T operands come straight from the row-major cache (a lane's 16 bytes are
// 8 consecutive head-dim elements of one token); V rows go through a
// wave-private LDS copy [32][D + 16] and are read back transposed. Register
// double-buffering: the next two pages load while the current two compute.
template <int D>
struct ContigGeom {
  static constexpr int NKS = D / 32;  // S^T k-steps (32 d each)
  static constexpr int NB = D / 16;   // PV output blocks (16 d each)
  // V: 16 rows x D of one page as 16-byte chunks per lane
  static constexpr int VROWREG = (16 * D * 2) / (64 * 16);
  static constexpr int kLdsBytesPerWave = 32 * (D + 16) * 2;
};

// Registers of one step (two pages): K and V as loaded from HBM.
template <int D>
struct ContigRegs {
  using G = ContigGeom<D>;
  u32x4 k[2][G::NKS];
  u32x4 vrow[2][G::VROWREG];
};

template <typename Tr, int D>
__global__ __launch_bounds__(kDecodeWgWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void decode_split_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ Kc, const uint16_t* __restrict__ Vc,
    uint16_t* __restrict__ O, float* __restrict__ ws_o, float* __restrict__ ws_lse, int Hq,
    int Hkv, int S_contig, int max_splits, int n_hc, long long total_waves, float scale_log2) {
  using vec8 = typename Tr::vec8;
  using vec4 = typename Tr::vec4;
  using vec2 = typename Tr::vec2;
  using G = ContigGeom<D>;
  constexpr int NKS = G::NKS, NB = G::NB;
  __shared__ __attribute__((aligned(16))) unsigned char lds[kDecodeWgWaves * G::kLdsBytesPerWave];

  // the wave index is uniform: readfirstlane keeps every per-wave quantity
  // derived from it (work item, page range, masks) in scalar registers
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const long long wid = (long long)blockIdx.x * kDecodeWgWaves + wave;
  if (wid >= total_waves) return;

  // ---- work item ----
  long long w = wid;
  const int split = (int)(w % max_splits);
  w /= max_splits;
  const int hc = (int)(w % n_hc);
  w /= n_hc;
  const int hk = (int)(w % Hkv);
  const int n = (int)(w / Hkv);
  const int Gq = Hq / Hkv;
  const int hq0 = hk * Gq + hc * 16;
  const int Gc = min(16, Gq - hc * 16);

  const int Lctx = S_contig;
  const int n_pages = (Lctx + kDecodePage - 1) / kDecodePage;
  const int n_splits = max(1, (n_pages + kPagesPerWave - 1) / kPagesPerWave);
  if (split >= n_splits) return;

  const int l16 = lane & 15, grp = lane >> 4;
  const int p_begin = split * kPagesPerWave;
  const int p_end = min(p_begin + kPagesPerWave, n_pages);
  const int n_steps = (p_end - p_begin + 1) / 2;  // 0 only for an empty context

  // ---- Q^T operand: lane (head g = l16, k-group grp) ----
  vec8 qv[NKS];
  {
    const uint16_t* qrow = Q + ((size_t)n * Hq + hq0 + l16) * D;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      if (l16 < Gc) {
        qv[ks] = *(const vec8*)(qrow + 32 * ks + 8 * grp);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[ks][e] = 0;
      }
    }
  }
  unsigned char* wlds = lds + wave * G::kLdsBytesPerWave;
  const size_t base = ((size_t)n * Hkv + hk) * (size_t)S_contig * D;
  const uint16_t* Kp = Kc + base;
  const uint16_t* Vp = Vc + base;

  // ---- HBM -> registers for one step ----
  auto load_step = [&](ContigRegs<D>& R, int step) {
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      const int page = p_begin + 2 * step + pp;
      const bool valid = page < p_end;
      const int tok = page * 16 + l16;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
        R.k[pp][ks] = (valid && tok < S_contig)
                          ? ld_stream<u32x4>(Kp + (size_t)tok * D + 32 * ks + 8 * grp)
                          : u32x4{0, 0, 0, 0};
      constexpr int CH = D / 8;
#pragma unroll
      for (int i = 0; i < G::VROWREG; ++i) {
        const int c = lane + 64 * i;
        const int vt = page * 16 + c / CH;
        R.vrow[pp][i] = (valid && vt < S_contig)
                            ? ld_stream<u32x4>(Vp + (size_t)vt * D + (c % CH) * 8)
                            : u32x4{0, 0, 0, 0};
      }
    }
  };

  f32x4 o[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf, l_run = 0.f;

  // ---- one step of attention on registers R ----
  auto compute_step = [&](const ContigRegs<D>& R, int step) {
    // stage the V rows into the wave's LDS
    {
      uint16_t* vl = (uint16_t*)wlds;
      constexpr int CH = D / 8;
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
#pragma unroll
        for (int i = 0; i < G::VROWREG; ++i) {
          const int c = lane + 64 * i;
          *(u32x4*)(vl + (16 * pp + c / CH) * (D + 16) + (c % CH) * 8) = R.vrow[pp][i];
        }
    }
    __builtin_amdgcn_wave_barrier();

    // S^T per page
    f32x4 s[2];
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      s[pp] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
        s[pp] = Tr::mfma16(__builtin_bit_cast(vec8, R.k[pp][ks]), qv[ks], s[pp]);
    }

    // online softmax over the step's 32 tokens
    const int pageA = p_begin + 2 * step;
    float x[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = s[0][r] * scale_log2;
      x[4 + r] = s[1][r] * scale_log2;
    }
    // tokens past the context (or the wave's last page) are masked; their V
    // slots are zeroed too
    const bool partial = (pageA + 2) * 16 > Lctx || pageA + 1 >= p_end;
    bool slot_ok[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tA = pageA * 16 + 4 * grp + r;
      slot_ok[r] = tA < Lctx;
      slot_ok[4 + r] = (tA + 16 < Lctx) && (pageA + 1 < p_end);
    }
    if (partial) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (!slot_ok[i]) x[i] = kNegInf;
    }
    float tmax = __builtin_fmaxf(max3(x[0], x[1], x[2]), max3(x[3], x[4], x[5]));
    tmax = max3(tmax, x[6], x[7]);
    tmax = pair16_max(tmax);
    tmax = pair32_max(tmax);
    const bool need = tmax > m_run + 8.0f;
    if (wave_any(need)) {
      const float m_new = __builtin_fmaxf(m_run, tmax);
      const float alpha = (m_new == kNegInf) ? 1.f : fast_exp2(m_run - m_new);
#pragma unroll
      for (int i = 0; i < NB; ++i) o[i] *= alpha;
      l_run *= alpha;
      m_run = m_new;
    }
    const float msub = (m_run == kNegInf) ? 0.f : m_run;
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = fast_exp2(x[i] - msub);
    l_run += (p[0] + p[1]) + (p[2] + p[3]) + (p[4] + p[5]) + (p[6] + p[7]);
    vec8 pa;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const vec2 ua = Tr::pack2(p[2 * j], p[2 * j + 1]);
      const vec2 ub = Tr::pack2(p[4 + 2 * j], p[4 + 2 * j + 1]);
      pa[2 * j] = ua[0];
      pa[2 * j + 1] = ua[1];
      pa[4 + 2 * j] = ub[0];
      pa[4 + 2 * j + 1] = ub[1];
    }

    // O += P V^T
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      // tr16: source lane (j = l16/4, c = l16%4) -> row (16pp + 4grp + j), col 16nb + 4c
      const uint16_t* vl = (const uint16_t*)wlds;
      const int row = 4 * grp + (l16 >> 2);
      const int col = 16 * nb + 4 * (l16 & 3);
      const vec4 lo = Tr::tr_read((const CA_LDS void*)(vl + row * (D + 16) + col));
      const vec4 hi = Tr::tr_read((const CA_LDS void*)(vl + (16 + row) * (D + 16) + col));
      vec8 bv = cat4<vec8, vec4>(lo, hi);
      if (partial) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (!slot_ok[i]) bv[i] = 0;
      }
      o[nb] = Tr::mfma16(pa, bv, o[nb]);
    }
    __builtin_amdgcn_wave_barrier();
  };

  // ---- the walk: register sets A and B alternate ----
  ContigRegs<D> A, B;
  if (n_steps > 0) load_step(A, 0);
  for (int step = 0; step < n_steps; step += 2) {
    if (step + 1 < n_steps) load_step(B, step + 1);
    compute_step(A, step);
    if (step + 1 >= n_steps) break;
    if (step + 2 < n_steps) load_step(A, step + 2);
    compute_step(B, step + 1);
  }

  // ---- totals over the 4 lanes of a head; m is already uniform ----
  l_run = pair16_sum(l_run);
  l_run = pair32_sum(l_run);
  const bool single = (n_splits == 1);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int g = 4 * grp + r;
    const float lg = __shfl(l_run, g, 64);
    const float mg = __shfl(m_run, g, 64);
    if (g >= Gc) continue;
    const float inv = (lg > 0.f) ? 1.f / lg : 0.f;
    const int hq = hq0 + g;
    if (single) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const vec2 pk = Tr::pack2(o[nb][r] * inv, 0.f);
        O[((size_t)n * Hq + hq) * D + 16 * nb + l16] = (uint16_t)(__builtin_bit_cast(uint32_t, pk) & 0xffffu);
      }
    } else {
      const size_t slot = ((size_t)n * Hq + hq) * max_splits + split;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) ws_o[slot * D + 16 * nb + l16] = o[nb][r] * inv;
      if (l16 == 0) ws_lse[slot] = (lg > 0.f) ? mg + __log2f(lg) : kNegInf;
    }
  }
}

// ---------------------------------------------------------------------------
// Paged decode with HBM -> LDS direct loads.
//
// Same math and work split as decode_split_kernel, but the pages travel from
// HBM straight into a per-wave LDS ring with global_load_lds_dwordx4 (each
// lane's 16 bytes land at ring slot + 16 * lane), so bytes in flight cost no
// VGPRs: a wave keeps kRing - 1 steps (two pages each, K and V) in flight.
// LDS is read with hand-issued ds_read instructions and the vector-memory
// counter is waited on explicitly (s_waitcnt vmcnt(N) with N = the loads
// issued after the step being consumed); the compiler's own conservative
// wait-for-everything before LDS reads would serialise the ring.
// Layouts in a ring slot: K pages as loaded ([D][16]; the 16-bit page's
// 16-byte chunks are XOR-swizzled on bit 3 of the chunk index by row-octet
// parity so the tr16 reads of lane groups 0/1 and 2/3 hit disjoint banks),
// V pages [D][16] with the 16-bit page's chunks swizzled too (chunk q at
// q ^ bit 4 of q): a 32-lane half of a V read takes the first or second 16
// bytes of 16 rows, 32 bytes apart, which without the swizzle put rows r
// and r + 8 on the same banks (a b64 read is conflict-free when each half
// covers 256 distinct bytes modulo 256). FP8 V rows are 16 bytes, and a
// b32 read of a lane's 4 tokens is 2-way conflicting (its halves need 32
// distinct dwords modulo 128 bytes from 16 rows, two dwords each), so the
// FP8 lanes read 8 bytes (tokens 8 (grp / 2) .. + 7: lane groups 0/1 and
// 2/3 read the same addresses, 16 rows x 8 bytes per half) and keep the
// dword of their own group.
// ---------------------------------------------------------------------------
// Ring depth (steps of one page, K and V, in flight per wave) and pages per
// split of the direct-load decode: 256 KB of K and V per split for both
// cache kinds (128 fp8 pages, two page-id registers per lane; 64 16-bit
// pages, one). A split's start (context length, block-table row, scales,
// filling the ring) is paid once per split: 128 fp8 pages measured +3.5 % on
// C4 over 64, while 128 16-bit pages leave C3 too few waves (-3 %). One page
// per step keeps a ring slot small (K + V of one page), so more waves fit a
// CU's LDS and more bytes are in flight per CU; the PV product then runs on
// 16x16x16 MFMAs, whose 4 k-values per lane are exactly the 4 tokens a lane
// holds. Page loads use the "nt" cache policy: every cache byte is read
// once per launch, so it is streamed rather than retained.
template <int KIND>
struct DmaCfg {
  // (rings of 3 / 2 fp8 steps or 2 16-bit steps, which let more waves share
  // a CU, measured within +-1 % on C4 / C3)
  // (the stream-K walk uses the same depths: deeper rings measured within
  // -0.5 % at head dim 128 and -3 .. +4 % at 64)
  static constexpr int kRing = KIND == kKindPagedFp8 ? 4 : 3;
  static constexpr int kPages = KIND == kKindPagedFp8 ? 128 : kPagesPerWave;
  // pages per ring fill of the stream-K walk
  static constexpr int kSkPages = 128;
  // decode_workspace_bytes sizes the partials for kPagesPerWave-page splits
  static_assert(kPages >= kPagesPerWave, "pages per split");
};
constexpr int kDmaPolicy = 2;  // global_load_lds cache policy bits: nt

// The wave's GQA group of query rows (Gc <= 16 heads from `qrow`, D each) as
// the B operand of S^T = K^T Q^T: lane (head l16, group grp) holds d = 32 ks
// + 8 grp .. + 7; rows past Gc are zero.
template <typename Tr, int D>
__device__ __forceinline__ void dma_load_q(const uint16_t* __restrict__ qrow, int Gc,
                                           typename Tr::vec8 (&qv)[D / 32]) {
  const int lane = threadIdx.x, l16 = lane & 15, grp = lane >> 4;
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
    if (l16 < Gc) {
      qv[ks] = *(const typename Tr::vec8*)(qrow + (size_t)l16 * D + 32 * ks + 8 * grp);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qv[ks][e] = 0;
    }
  }
}

// One wave's walk over pages [p_begin, p_end) (at most PAGES)
// of one (sequence, kv head hk) whose block-table row is `bt_row`. The
// online-softmax state (o, m_run, l_run) is carried in and out, so a
// context can be walked in several calls; the ring is filled at the start
// and drained at the end of each call.
template <typename Tr, int D, int KIND, int RING = DmaCfg<KIND>::kRing,
          int PAGES = DmaCfg<KIND>::kPages>
__device__ __forceinline__ void dma_walk(const typename Tr::vec8 (&qv)[D / 32], f32x4 (&o)[D / 16],
                                         float& m_run, float& l_run, unsigned char* ring,
                                         const void* __restrict__ Kc, const void* __restrict__ Vc,
                                         const float* __restrict__ k_scale,
                                         const float* __restrict__ v_scale, int per_block,
                                         const int32_t* __restrict__ bt_row, int Hkv, int hk,
                                         int num_blocks, int p_begin, int p_end, int Lctx,
                                         float scale_log2, const unsigned char* dummy) {
  using vec8 = typename Tr::vec8;
  using vec4 = typename Tr::vec4;
  constexpr int NKS = D / 32, NB = D / 16;
  constexpr bool FP8 = KIND == kKindPagedFp8;
  constexpr int ELEM = FP8 ? 1 : 2;
  constexpr int CHUNK = D * 16 * ELEM;        // bytes of one (page, head) chunk
  constexpr int NDMA = CHUNK / 1024;          // 16 B x 64 lanes per load
  constexpr int STAGE = 2 * CHUNK;            // K and V of the step's page
  constexpr int DPS = 2 * NDMA;               // loads per step
  constexpr int KRD = FP8 ? NKS : 2 * NKS;    // LDS reads for one page's K^T operands
  constexpr int PB = PAGES / 64;              // page-id registers per lane
  static_assert(PAGES % 64 == 0 && PB <= 2, "pages per split");
  static_assert((RING - 1) * DPS <= 63, "vmcnt range");

  const int lane = threadIdx.x;
  const int l16 = lane & 15, grp = lane >> 4;
  const int n_steps = p_end - p_begin;

  // page ids and per-page scales: lane j of register b holds page
  // p_begin + 64 b + j; read back for page index i (uniform) with lane_val
  int pid_lane[PB];
  float ksc_lane[PB], vsc_lane[PB];
#pragma unroll
  for (int pb = 0; pb < PB; ++pb) {
    const int page = p_begin + 64 * pb + lane;
    pid_lane[pb] = 0;
    ksc_lane[pb] = vsc_lane[pb] = 1.f;
    if (page < p_end) {
      pid_lane[pb] = bt_row[page];
      pid_lane[pb] = min(max(pid_lane[pb], 0), num_blocks - 1);
    }
    if (FP8) {
      if (per_block) {
        if (page < p_end) {
          ksc_lane[pb] = k_scale[(size_t)pid_lane[pb] * Hkv + hk];
          vsc_lane[pb] = v_scale[(size_t)pid_lane[pb] * Hkv + hk];
        }
      } else {
        ksc_lane[pb] = k_scale[hk];
        vsc_lane[pb] = v_scale[hk];
      }
    }
  }
  auto lane_val = [&](const auto (&r)[PB], int i) CA_INLINE {
    const auto v = (PB > 1 && i >= 64) ? r[PB - 1] : r[0];
    return __builtin_bit_cast(std::remove_const_t<std::remove_reference_t<decltype(r[0])>>,
                              __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), i & 63));
  };

  // source byte offset of this lane's 16 bytes for load i of a K chunk
  auto k_src = [&](int i) -> int {
    const int p = 64 * i + lane;  // physical 16-byte slot in LDS
    if (FP8) return 16 * p;
    return 16 * (p ^ (((p >> 4) & 1) << 3));
  };
  // source offset of this lane's 16 bytes in each 1 KB of a V chunk
  const int v_src = 16 * (FP8 ? lane : lane ^ ((lane >> 4) & 1));
  auto issue_step = [&](int step, int slot) {
    unsigned char* base = ring + slot * STAGE;
    const bool valid = step < n_steps;
    const int pid = lane_val(pid_lane, valid ? step : 0);
    const size_t chunk = ((size_t)pid * Hkv + hk) * (size_t)CHUNK;
    const unsigned char* kp = (const unsigned char*)Kc + chunk;
    const unsigned char* vp = (const unsigned char*)Vc + chunk;
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      dma16<kDmaPolicy>(valid ? kp + k_src(i) : dummy, (CA_LDS void*)(base + 1024 * i));
      dma16<kDmaPolicy>(valid ? vp + 1024 * i + v_src : dummy,
                        (CA_LDS void*)(base + CHUNK + 1024 * i));
    }
  };

  // per-lane LDS read offsets inside a page's K / V chunk
  uint32_t k_lo, k_hi;
  if (FP8) {
    k_lo = 16 * (8 * grp + (l16 >> 1)) + 8 * (l16 & 1);
    k_hi = 0;
  } else {
    const int c = l16 & 3, j = l16 >> 2, par = grp & 1;
    k_lo = 16 * (16 * grp + 8 * par + 2 * j + (c >> 1)) + 8 * (c & 1);
    k_hi = 16 * (16 * grp + 8 * (1 - par) + 2 * j + (c >> 1)) + 8 * (c & 1);
  }
  // V: lane (d = l16, token group grp) needs tokens 4 grp .. 4 grp + 3 of row d
  // (FP8: the 8 bytes of tokens 8 (grp / 2) .. + 7, then its own dword)
  const uint32_t v_off = FP8 ? (uint32_t)(16 * l16 + 8 * (grp >> 1))
                             : (uint32_t)(16 * ((2 * l16 + (grp >> 1)) ^ ((l16 >> 3) & 1)) + 8 * (grp & 1));
  const uint32_t ring0 = lds_off(ring);

  // RING steps in flight from the start; a slot is refilled as soon as its
  // LDS reads have returned, so RING steps stay in flight during the math
#pragma unroll
  for (int st = 0; st < RING; ++st) issue_step(st, st);
  int slot = 0;
  for (int step = 0; step < n_steps; ++step) {
    wait_vmcnt<(RING - 1) * DPS>();  // this step's loads are the oldest outstanding
    const uint32_t kb = ring0 + slot * STAGE;
    const uint32_t vb = kb + CHUNK + v_off;

    // ---- LDS -> operands ----
    u32x2 kraw[KRD];
    u32x2 v8r[FP8 ? NB : 1];
    u32x2 v16r[FP8 ? 1 : NB];
    if (FP8) {
      const uint32_t a = kb + k_lo;
      kraw[0] = lds_read_tr8<0>(a);
      if (NKS > 1) kraw[1 % KRD] = lds_read_tr8<512>(a);
      if (NKS > 2) kraw[2 % KRD] = lds_read_tr8<1024>(a);
      if (NKS > 3) kraw[3 % KRD] = lds_read_tr8<1536>(a);
#define CA_V8(NBI) if (NBI < NB) v8r[NBI % NB] = lds_read_b64<256 * NBI>(vb);
      CA_V8(0) CA_V8(1) CA_V8(2) CA_V8(3) CA_V8(4) CA_V8(5) CA_V8(6) CA_V8(7)
#undef CA_V8
    } else {
      const uint32_t alo = kb + k_lo, ahi = kb + k_hi;
      kraw[0] = lds_read_tr16<0>(alo);
      kraw[1] = lds_read_tr16<0>(ahi);
      if (NKS > 1) { kraw[2 % KRD] = lds_read_tr16<1024>(alo); kraw[3 % KRD] = lds_read_tr16<1024>(ahi); }
      if (NKS > 2) { kraw[4 % KRD] = lds_read_tr16<2048>(alo); kraw[5 % KRD] = lds_read_tr16<2048>(ahi); }
      if (NKS > 3) { kraw[6 % KRD] = lds_read_tr16<3072>(alo); kraw[7 % KRD] = lds_read_tr16<3072>(ahi); }
#define CA_V16(NBI) if (NBI < NB) v16r[NBI % NB] = lds_read_b64<512 * NBI>(vb);
      CA_V16(0) CA_V16(1) CA_V16(2) CA_V16(3) CA_V16(4) CA_V16(5) CA_V16(6) CA_V16(7)
#undef CA_V16
    }
    wait_lgkm0();
#pragma unroll
    for (int i = 0; i < KRD; ++i) after_wait(kraw[i]);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      if (FP8) after_wait(v8r[i % (FP8 ? NB : 1)]);
      else after_wait(v16r[i % (FP8 ? 1 : NB)]);
    }
    issue_step(step + RING, slot);  // the slot's data is in registers now

    // ---- S^T of the page ----
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      vec8 a;
      if (FP8) {
        a = fp8x8_to<Tr>(kraw[ks % KRD][0], kraw[ks % KRD][1]);
      } else {
        const u32x4 t = {kraw[(2 * ks) % KRD][0], kraw[(2 * ks) % KRD][1],
                         kraw[(2 * ks + 1) % KRD][0], kraw[(2 * ks + 1) % KRD][1]};
        a = __builtin_bit_cast(vec8, t);
      }
      s = Tr::mfma16(a, qv[ks], s);
    }

    // ---- online softmax over the page's 16 tokens ----
    const int page0 = p_begin + step;
    float c = scale_log2, vs = 1.f;
    if (FP8) {
      c *= lane_val(ksc_lane, step);
      vs = lane_val(vsc_lane, step);
    }
    float x[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) x[r] = s[r] * c;
    // tokens past the context are masked; their V slots are zeroed too, so
    // stale cache bytes (NaN patterns included) in a partially filled page
    // cannot reach the PV product
    const bool partial = (page0 + 1) * 16 > Lctx;
    bool slot_ok[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) slot_ok[r] = page0 * 16 + 4 * grp + r < Lctx;
    if (partial) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (!slot_ok[i]) x[i] = kNegInf;
    }
    float tmax = max3(x[0], x[1], __builtin_fmaxf(x[2], x[3]));
    tmax = pair16_max(tmax);
    tmax = pair32_max(tmax);
    const bool need = tmax > m_run + 8.0f;
    if (wave_any(need)) {
      const float m_new = __builtin_fmaxf(m_run, tmax);
      const float alpha = (m_new == kNegInf) ? 1.f : fast_exp2(m_run - m_new);
#pragma unroll
      for (int i = 0; i < NB; ++i) o[i] *= alpha;
      l_run *= alpha;
      m_run = m_new;
    }
    const float msub = (m_run == kNegInf) ? 0.f : m_run;
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = fast_exp2(x[i] - msub);
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) psum += p[i];
    l_run += psum;
    // P operand (v scale folded in): the lane's 4 tokens (16x16x16)
    u32x2 pw;
    pw[0] = __builtin_bit_cast(uint32_t, Tr::pack2(p[0] * vs, p[1] * vs));
    pw[1] = __builtin_bit_cast(uint32_t, Tr::pack2(p[2] * vs, p[3] * vs));

    // ---- O += P V^T ----
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      u32x2 bw;
      if (FP8) {
        const uint32_t v = (grp & 1) ? v8r[nb % (FP8 ? NB : 1)][1] : v8r[nb % (FP8 ? NB : 1)][0];
        bw[0] = __builtin_bit_cast(uint32_t, Fp8Conv<Tr>::template cvt<false>(v));
        bw[1] = __builtin_bit_cast(uint32_t, Fp8Conv<Tr>::template cvt<true>(v));
      } else {
        bw[0] = v16r[nb % (FP8 ? 1 : NB)][0];
        bw[1] = v16r[nb % (FP8 ? 1 : NB)][1];
      }
      if (partial) {
        // zero masked token slots: 16-bit halves of the operand dwords
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (!slot_ok[i]) bw[i >> 1] &= (i & 1) ? 0x0000ffffu : 0xffff0000u;
      }
      o[nb] = Tr::mfma16k16(__builtin_bit_cast(vec4, pw), __builtin_bit_cast(vec4, bw), o[nb]);
    }
    slot = (slot == RING - 1) ? 0 : slot + 1;
  }
  wait_vmcnt<0>();  // no load may still target this workgroup's LDS when it exits
}

// The wave's Gc query heads normalised by their sums: written to the output
// (`out_rows`, head g at + g D) or, when out_rows is null, as a partial for a
// merge (o / l at po + g po_stride, log2-sum-exp at plse + g plse_stride).
template <typename Tr, int D>
__device__ __forceinline__ void dma_finish(const f32x4 (&o)[D / 16], float m_run, float l_run,
                                           int Gc, uint16_t* __restrict__ out_rows,
                                           float* __restrict__ po, size_t po_stride,
                                           float* __restrict__ plse, size_t plse_stride) {
  using vec2 = typename Tr::vec2;
  constexpr int NB = D / 16;
  const int lane = threadIdx.x, l16 = lane & 15, grp = lane >> 4;
  l_run = pair16_sum(l_run);
  l_run = pair32_sum(l_run);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int g = 4 * grp + r;
    const float lg = __shfl(l_run, g, 64);
    const float mg = __shfl(m_run, g, 64);
    if (g >= Gc) continue;
    const float inv = (lg > 0.f) ? 1.f / lg : 0.f;
    if (out_rows) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const vec2 pk = Tr::pack2(o[nb][r] * inv, 0.f);
        out_rows[(size_t)g * D + 16 * nb + l16] = (uint16_t)(__builtin_bit_cast(uint32_t, pk) & 0xffffu);
      }
    } else {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) po[g * po_stride + 16 * nb + l16] = o[nb][r] * inv;
      if (l16 == 0) plse[g * plse_stride] = (lg > 0.f) ? mg + __log2f(lg) : kNegInf;
    }
  }
}

// Split grid: one wave per split of DmaCfg<KIND>::kPages pages of one
// (sequence, kv head, query-head chunk of <= 16).
template <typename Tr, int D, int KIND>
__global__ __launch_bounds__(64) void decode_dma_kernel(
    const uint16_t* __restrict__ Q, const void* __restrict__ Kc, const void* __restrict__ Vc,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale, int per_block,
    const int32_t* __restrict__ block_tables, const int32_t* __restrict__ context_lens,
    uint16_t* __restrict__ O, float* __restrict__ ws_o, float* __restrict__ ws_lse, int Hq,
    int Hkv, int max_blocks, int num_blocks, int max_splits, int n_hc, float scale_log2) {
  constexpr int NKS = D / 32, NB = D / 16;
  constexpr int STAGE = 2 * D * 16 * (KIND == kKindPagedFp8 ? 1 : 2);
  constexpr int kDmaPages = DmaCfg<KIND>::kPages;
  __shared__ __attribute__((aligned(1024))) unsigned char ring[DmaCfg<KIND>::kRing * STAGE];

  int w = blockIdx.x;
  // split index outermost, counted from each sequence's end: the waves of
  // splits before a sequence's start (none exist) come first and retire at
  // once, and every sequence's last (partial) split is in the final group
  const int per_split = (int)(gridDim.x / max_splits);
  const int from_end = max_splits - 1 - w / per_split;
  w %= per_split;
  const int hc = w % n_hc;
  w /= n_hc;
  const int hk = w % Hkv;
  const int n = w / Hkv;
  const int Gq = Hq / Hkv;
  const int hq0 = hk * Gq + hc * 16;
  const int Gc = min(16, Gq - hc * 16);
  const int Lctx = min(max(0, context_lens[n]), max_blocks * kDecodePage);
  const int n_pages = (Lctx + kDecodePage - 1) / kDecodePage;
  const int n_splits = max(1, (n_pages + kDmaPages - 1) / kDmaPages);
  const int split = n_splits - 1 - from_end;
  if (split < 0) return;
  const int p_begin = split * kDmaPages;
  const int p_end = min(p_begin + kDmaPages, n_pages);

  typename Tr::vec8 qv[NKS];
  dma_load_q<Tr, D>(Q + ((size_t)n * Hq + hq0) * D, Gc, qv);
  f32x4 o[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf, l_run = 0.f;
  dma_walk<Tr, D, KIND>(qv, o, m_run, l_run, ring, Kc, Vc, k_scale, v_scale, per_block,
                        block_tables + (size_t)n * max_blocks, Hkv, hk, num_blocks, p_begin, p_end,
                        Lctx, scale_log2, (const unsigned char*)Q);
  if (n_splits == 1) {
    dma_finish<Tr, D>(o, m_run, l_run, Gc, O + ((size_t)n * Hq + hq0) * D, nullptr, 0, nullptr, 0);
  } else {
    const size_t sl = ((size_t)n * Hq + hq0) * max_splits + split;
    dma_finish<Tr, D>(o, m_run, l_run, Gc, nullptr, ws_o + sl * D, (size_t)max_splits * D,
                      ws_lse + sl, (size_t)max_splits);
  }
}

// ---------------------------------------------------------------------------
// Balanced ("stream-K") paged decode. The work units are (sequence, kv head,
// query-head chunk, page) in that order (a sequence's units are its pages
// times its Hkv * n_hc segments); wave w of W takes units [w T / W,
// (w + 1) T / W) of the T in the launch, so every wave streams the same
// number of pages whatever the context lengths are; W is one wave per SIMD
// of the device, all resident at once (each wave pays its start once). A wave
// walks its range segment by segment (a segment: one (sequence, kv head,
// chunk), walked kPages pages per ring fill); a segment inside the range is
// written as output, one cut by the range's start or end as a partial (at
// most two per wave: slot 0 for the first piece, 1 for the last), which
// decode_sk_merge_kernel combines. Every wave scans the context lengths
// itself to find where its range starts (N <= kSkMaxSeqs, 16 per lane);
// wave 0 also stores the inclusive prefix of units per sequence for the
// merge.
// Workspace: [W][2][GMAX] x D floats of o / l, [W][2][GMAX] floats of
// log2-sum-exp, then N ints of prefix (GMAX = min(16, Hq / Hkv)).
// ---------------------------------------------------------------------------
constexpr int kSkMaxSeqs = 1024;
constexpr int kSkMinPages = 16;   // fewer waves when the launch has < 16 pages each

__device__ __forceinline__ int sk_waves_used(int grid, int T) {
  return max(1, min(grid, T / kSkMinPages));
}

template <typename Tr, int D, int KIND>
__global__ __launch_bounds__(64) void decode_sk_kernel(
    const uint16_t* __restrict__ Q, const void* __restrict__ Kc, const void* __restrict__ Vc,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale, int per_block,
    const int32_t* __restrict__ block_tables, const int32_t* __restrict__ context_lens,
    uint16_t* __restrict__ O, float* __restrict__ ws_o, float* __restrict__ ws_lse,
    int32_t* __restrict__ ws_prefix, int N, int Hq, int Hkv, int max_blocks, int num_blocks,
    int n_hc, float scale_log2) {
  constexpr int NKS = D / 32, NB = D / 16;
  constexpr int STAGE = 2 * D * 16 * (KIND == kKindPagedFp8 ? 1 : 2);
  constexpr int kDmaPages = DmaCfg<KIND>::kSkPages;
  constexpr int NCH = kSkMaxSeqs / 64;
  __shared__ __attribute__((aligned(1024))) unsigned char ring[DmaCfg<KIND>::kRing * STAGE];

  const int lane = threadIdx.x;
  const int segs = Hkv * n_hc;
  const int max_tokens = max_blocks * kDecodePage;
  // inclusive prefix of units over sequences: sequence 64 c + lane in incl[c]
  // (lanes and chunks past N hold the total)
  int incl[NCH];
  int carry = 0;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    incl[c] = carry;
    if (64 * c < N) {
      const int n = 64 * c + lane;
      int u = 0;
      if (n < N) u = ((min(max(0, context_lens[n]), max_tokens) + kDecodePage - 1) / kDecodePage) * segs;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(u, off, 64);
        if (lane >= off) u += t;
      }
      incl[c] = carry + u;
      carry = __shfl(incl[c], 63, 64);
    }
  }
  const int T = carry;
  if (blockIdx.x == 0) {
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      if (64 * c + lane < N) ws_prefix[64 * c + lane] = incl[c];
  }
  if (T == 0) return;
  const int W = sk_waves_used((int)gridDim.x, T);
  const int w = blockIdx.x;
  if (w >= W) return;
  const int a = (int)((long long)w * T / W), b = (int)((long long)(w + 1) * T / W);
  if (a == b) return;

  // sequence holding unit a: the number of sequences whose units end at or before it
  int n = 0;
#pragma unroll
  for (int c = 0; c < NCH; ++c) n += __popcll(__ballot(incl[c] <= a));
  auto incl_at = [&](int i) CA_INLINE {   // i uniform, < kSkMaxSeqs
    int v = 0;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      if (c == (i >> 6)) v = incl[c];
    return __builtin_amdgcn_readlane(v, i & 63);
  };
  // from here on the prefix comes from the lengths (incl[] is dead in the walk)
  int exc = n ? incl_at(n - 1) : 0, inc = incl_at(n);
  auto seq_units = [&](int i) CA_INLINE {
    return ((min(max(0, context_lens[i]), max_tokens) + kDecodePage - 1) / kDecodePage) * segs;
  };

  const int Gq = Hq / Hkv;
  const int GMAX = min(16, Gq);
  typename Tr::vec8 qv[NKS];
  f32x4 o[NB];
  int u = a;
  while (u < b) {
    const int pages = (inc - exc) / segs;   // >= 1: sequence n holds unit u
    const int r = u - exc;
    const int seg = r / pages, p0 = r - seg * pages;
    const int len = min(b - u, pages - p0);
    const int hk = seg / n_hc, hc = seg - hk * n_hc;
    const int hq0 = hk * Gq + hc * 16, Gc = min(16, Gq - hc * 16);
    const int Lctx = min(max(0, context_lens[n]), max_tokens);
    dma_load_q<Tr, D>(Q + ((size_t)n * Hq + hq0) * D, Gc, qv);
#pragma unroll
    for (int i = 0; i < NB; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = kNegInf, l_run = 0.f;
    // ring fills at multiples of kPages pages of the context (so waves that
    // share a segment do not refill in step)
    for (int p = p0; p < p0 + len;) {
      const int pe = min(p0 + len, (p / kDmaPages + 1) * kDmaPages);
      dma_walk<Tr, D, KIND, DmaCfg<KIND>::kRing, kDmaPages>(
          qv, o, m_run, l_run, ring, Kc, Vc, k_scale, v_scale, per_block,
          block_tables + (size_t)n * max_blocks, Hkv, hk, num_blocks, p, pe, Lctx, scale_log2,
          (const unsigned char*)Q);
      p = pe;
    }
    if (p0 == 0 && len == pages) {
      dma_finish<Tr, D>(o, m_run, l_run, Gc, O + ((size_t)n * Hq + hq0) * D, nullptr, 0, nullptr, 0);
    } else {
      const size_t row = (size_t)(2 * w + (u == a ? 0 : 1)) * GMAX;
      dma_finish<Tr, D>(o, m_run, l_run, Gc, nullptr, ws_o + row * D, D, ws_lse + row, 1);
    }
    u += len;
    if (u < b && u == inc) {   // the sequence is done: the next one with units
      do {
        ++n;
        exc = inc;
        inc = exc + seq_units(n);
      } while (inc == exc);
    }
  }
}

// Combines n_parts partials (o / l rows and log2-sum-exp values, partial k at
// row idx(k)) into output row `orow`: o = sum_k 2^(lse_k - M) o_k / sum_k
// 2^(lse_k - M). Each lane owns D/64 output elements. Bound by memory
// latency, not bytes: the first kMergeAhead partials are loaded together with
// the log2-sum-exp values, before their maximum is known, so up to
// kMergeAhead partials take one round trip; the sum runs over the partials in
// order either way.
constexpr int kMergeAhead = 16;
template <typename Tr, int D, typename Idx>
__device__ __forceinline__ void merge_rows(int n_parts, Idx idx, const float* __restrict__ ws_o,
                                           const float* __restrict__ ws_lse, void* __restrict__ O,
                                           size_t orow) {
  constexpr int PER = D / 64;
  const int lane = threadIdx.x;
  const float lse0 = lane < n_parts ? ws_lse[idx(lane)] : kNegInf;  // partial `lane`
  const int n_ahead = min(kMergeAhead, n_parts);
  float part[kMergeAhead][PER];
#pragma unroll
  for (int j = 0; j < kMergeAhead; ++j)
    if (j < n_ahead) {
#pragma unroll
      for (int i = 0; i < PER; ++i) part[j][i] = ws_o[idx(j) * D + lane * PER + i];
    }
  float M = lse0;
  for (int s = lane + 64; s < n_parts; s += 64) M = __builtin_fmaxf(M, ws_lse[idx(s)]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) M = __builtin_fmaxf(M, __shfl_xor(M, off, 64));
  float wsum = 0.f;
  float acc[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) acc[i] = 0.f;
  if (M != kNegInf) {
    for (int s0 = 0; s0 < n_parts; s0 += 64) {
      const int s = s0 + lane;
      const float lse = s0 == 0 ? lse0 : (s < n_parts) ? ws_lse[idx(s)] : kNegInf;
      const float wl = (lse == kNegInf) ? 0.f : fast_exp2(lse - M);
      const int cnt = min(64, n_parts - s0);
      int j0 = 0;
      if (s0 == 0) {
#pragma unroll
        for (int j = 0; j < kMergeAhead; ++j)
          if (j < n_ahead) {
            const float wj = __shfl(wl, j, 64);
            wsum += wj;
#pragma unroll
            for (int i = 0; i < PER; ++i) acc[i] += wj * part[j][i];
          }
        j0 = n_ahead;
      }
#pragma unroll 4
      for (int j = j0; j < cnt; ++j) {
        const float wj = __shfl(wl, j, 64);
        wsum += wj;
        const float* src = ws_o + idx(s0 + j) * D + lane * PER;
#pragma unroll
        for (int i = 0; i < PER; ++i) acc[i] += wj * src[i];
      }
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) Tr::store(O, orow + lane * PER + i, acc[i] * inv);
}

// Split-grid merge: one wave per (sequence, query head) with more than one
// split; the partials of split s at [n][hq][s].
template <typename Tr, int D>
__global__ __launch_bounds__(64) void decode_merge_kernel(
    const int32_t* __restrict__ context_lens, int max_tokens, const float* __restrict__ ws_o,
    const float* __restrict__ ws_lse, void* __restrict__ O, int Hq, int max_splits,
    int pages_per_split) {
  const int n = blockIdx.x / Hq, hq = blockIdx.x % Hq;
  const int Lctx = context_lens ? min(max(0, context_lens[n]), max_tokens) : max_tokens;
  const int n_pages = (Lctx + kDecodePage - 1) / kDecodePage;
  const int n_splits = (n_pages + pages_per_split - 1) / pages_per_split;
  if (n_splits <= 1) return;
  const size_t slot0 = ((size_t)n * Hq + hq) * max_splits;
  merge_rows<Tr, D>(n_splits, [&](int k) CA_INLINE { return slot0 + k; }, ws_o, ws_lse, O,
                    ((size_t)n * Hq + hq) * D);
}

// Stream-K merge: one wave per (sequence, query head). Its segment's units
// [u0, u1) were walked by waves wave_of(u0) .. wave_of(u1 - 1); a segment of
// one wave was written by it, an empty one (no context) is written here as
// zeros, any other is merged from its waves' partials (the first wave's slot
// 1 when the segment is not where that wave starts, slot 0 otherwise).
template <typename Tr, int D>
__global__ __launch_bounds__(64) void decode_sk_merge_kernel(
    const int32_t* __restrict__ ws_prefix, const float* __restrict__ ws_o,
    const float* __restrict__ ws_lse, void* __restrict__ O, int N, int Hq, int Hkv, int n_hc,
    int grid) {
  constexpr int PER = D / 64;
  const int n = blockIdx.x / Hq, hq = blockIdx.x % Hq;
  const int lane = threadIdx.x;
  const int Gq = Hq / Hkv, GMAX = min(16, Gq);
  const int hk = hq / Gq, j = hq - hk * Gq, hc = j / 16, g = j - 16 * hc;
  const int segs = Hkv * n_hc;
  const int exc = n ? ws_prefix[n - 1] : 0, inc = ws_prefix[n];
  const int pages = (inc - exc) / segs;
  const size_t orow = ((size_t)n * Hq + hq) * D;
  if (pages == 0) {
#pragma unroll
    for (int i = 0; i < PER; ++i) Tr::store(O, orow + lane * PER + i, 0.f);
    return;
  }
  const int T = ws_prefix[N - 1];
  const int W = sk_waves_used(grid, T);
  const int u0 = exc + (hk * n_hc + hc) * pages, u1 = u0 + pages;
  auto wave_of = [&](int u) { return (int)(((long long)(u + 1) * W - 1) / T); };
  const int w0 = wave_of(u0), w1 = wave_of(u1 - 1);
  if (w0 == w1) return;
  const int s0 = ((long long)w0 * T / W < u0) ? 1 : 0;
  merge_rows<Tr, D>(w1 - w0 + 1,
                    [&](int k) CA_INLINE { return (size_t)(2 * (w0 + k) + (k == 0 ? s0 : 0)) * GMAX + g; },
                    ws_o, ws_lse, O, orow);
}

// Bytes of split partials for max_splits splits per (sequence, query head):
// [N][Hq][max_splits] x D floats of o / l, then [N][Hq][max_splits] floats
// of log2-sum-exp; none when every context fits one split.
static size_t split_partials_bytes(int N, int Hq, int D, int max_splits) {
  if (max_splits <= 1) return 0;
  return (size_t)N * Hq * max_splits * (size_t)(D + 1) * sizeof(float);
}

size_t decode_workspace_bytes(int N, int Hq, int D, int max_tokens) {
  // rounded up without forming max_tokens + page - 1 (no overflow near INT_MAX)
  const int pages = max_tokens / kDecodePage + (max_tokens % kDecodePage != 0);
  return split_partials_bytes(N, Hq, D, pages / kPagesPerWave + (pages % kPagesPerWave != 0));
}

// Waves per CU of a stream-K launch. Every wave streams the same bytes, so a
// CU must hold a multiple of four for its SIMDs to finish together; one per
// SIMD measured best, except where a page step is only 2 KB (FP8 at head dim
// 64): there one wave cannot cover its own per-step latency, and two per
// SIMD run 5632-6006 GB/s against 4375-4611 (reference-grid shapes).
template <int KIND, int D>
constexpr int sk_waves_per_cu() {
  return 2 * D * 16 * (KIND == kKindPagedFp8 ? 1 : 2) < 4096 ? 8 : 4;
}

// Grid of the stream-K decode on the current device (0 if unknown), cached
// per device like device_cus.
template <typename Tr, int D, int KIND>
static int sk_grid() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int g = cached[dev].load(std::memory_order_relaxed);
  if (g == 0) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void*>(&decode_sk_kernel<Tr, D, KIND>), 64, 0) !=
        hipSuccess)
      return 0;
    g = std::min(per_cu, sk_waves_per_cu<KIND, D>()) * device_cus();
    cached[dev].store(g, std::memory_order_relaxed);
  }
  return g;
}

static size_t sk_partials_bytes(int grid, int N, int Gq, int D) {
  return (size_t)2 * grid * std::min(16, Gq) * (size_t)(D + 1) * sizeof(float) +
         (size_t)N * sizeof(int32_t);
}

// How a paged decode launch splits its work: stream-K (grid > 0) when its
// partials fit the workspace every caller provides (decode_workspace_bytes)
// and the sequences fit the prefix registers; otherwise the split grid.
struct PagedPlan {
  int grid = 0;          // stream-K waves, 0 for the split grid
  int max_splits = 1;    // split grid: splits of the longest context
  size_t bytes = 0;      // partials the launch writes
};
template <typename Tr, int D, int KIND>
static PagedPlan paged_plan(int N, int Hq, int Hkv, int max_blocks) {
  PagedPlan p;
  constexpr int kPages = DmaCfg<KIND>::kPages;
  p.max_splits = std::max(1, max_blocks / kPages + (max_blocks % kPages != 0));
  const int Gq = Hq / Hkv;
  const int n_hc = (Gq + 15) / 16;
  if (p.max_splits > 1 && N <= kSkMaxSeqs &&
      (long long)N * max_blocks * Hkv * n_hc <= (long long)INT_MAX) {
    const int g = sk_grid<Tr, D, KIND>();
    const size_t need = sk_partials_bytes(g, N, Gq, D);
    if (g > 0 && need <= decode_workspace_bytes(N, Hq, D, max_blocks * kDecodePage)) {
      p.grid = g;
      p.bytes = need;
      return p;
    }
  }
  p.bytes = split_partials_bytes(N, Hq, D, p.max_splits);
  return p;
}

template <typename Tr, int D, int KIND>
static hipError_t launch_paged_decode_t(const void* q, const void* kc, const void* vc,
                                        const float* k_scale, const float* v_scale, int per_block,
                                        const int32_t* bt, const int32_t* lens, void* out, int N,
                                        int Hq, int Hkv, int max_blocks, int num_blocks,
                                        float scale, void* ws, size_t ws_bytes,
                                        hipStream_t stream) {
  const int max_tokens = max_blocks * kDecodePage;
  const int Gq = Hq / Hkv;
  const int n_hc = (Gq + 15) / 16;
  const PagedPlan plan = paged_plan<Tr, D, KIND>(N, Hq, Hkv, max_blocks);
  if (ws_bytes < plan.bytes) return hipErrorInvalidValue;
  if (plan.grid > 0) {
    const size_t rows = (size_t)2 * plan.grid * std::min(16, Gq);
    float* ws_o = (float*)ws;
    float* ws_lse = ws_o + rows * D;
    int32_t* ws_prefix = (int32_t*)(ws_lse + rows);
    hipLaunchKernelGGL((decode_sk_kernel<Tr, D, KIND>), dim3((unsigned)plan.grid), dim3(64), 0,
                       stream, (const uint16_t*)q, kc, vc, k_scale, v_scale, per_block, bt, lens,
                       (uint16_t*)out, ws_o, ws_lse, ws_prefix, N, Hq, Hkv, max_blocks,
                       num_blocks, n_hc, scale * kLog2e);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((decode_sk_merge_kernel<Tr, D>), dim3((unsigned)(N * Hq)), dim3(64), 0,
                       stream, ws_prefix, ws_o, ws_lse, out, N, Hq, Hkv, n_hc, plan.grid);
    return hipGetLastError();
  }
  const int max_splits = plan.max_splits;
  float* ws_o = (float*)ws;
  float* ws_lse = plan.bytes ? ws_o + (size_t)N * Hq * max_splits * D : nullptr;
  const long long total_waves = (long long)N * Hkv * n_hc * max_splits;
  if (total_waves == 0) return hipSuccess;
  if (total_waves > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((decode_dma_kernel<Tr, D, KIND>), dim3((unsigned)total_waves), dim3(64), 0,
                     stream, (const uint16_t*)q, kc, vc, k_scale, v_scale, per_block, bt, lens,
                     (uint16_t*)out, ws_o, ws_lse, Hq, Hkv, max_blocks, num_blocks, max_splits,
                     n_hc, scale * kLog2e);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || max_splits <= 1) return e;
  hipLaunchKernelGGL((decode_merge_kernel<Tr, D>), dim3((unsigned)(N * Hq)), dim3(64), 0, stream,
                     lens, max_tokens, ws_o, ws_lse, out, Hq, max_splits, DmaCfg<KIND>::kPages);
  return hipGetLastError();
}

template <typename Tr, int D>
static hipError_t launch_contig_decode_t(const void* q, const void* k, const void* v, void* out,
                                         int N, int Hq, int Hkv, int S, float scale, void* ws,
                                         size_t ws_bytes, hipStream_t stream) {
  const int pages = (S + kDecodePage - 1) / kDecodePage;
  const int max_splits = max(1, (pages + kPagesPerWave - 1) / kPagesPerWave);
  const int Gq = Hq / Hkv;
  const int n_hc = (Gq + 15) / 16;
  const size_t need = decode_workspace_bytes(N, Hq, D, S);
  if (ws_bytes < need) return hipErrorInvalidValue;
  float* ws_o = (float*)ws;
  float* ws_lse = need ? ws_o + (size_t)N * Hq * max_splits * D : nullptr;
  const long long total_waves = (long long)N * Hkv * n_hc * max_splits;
  if (total_waves == 0) return hipSuccess;
  const long long grid = (total_waves + kDecodeWgWaves - 1) / kDecodeWgWaves;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((decode_split_kernel<Tr, D>), dim3((unsigned)grid), dim3(kDecodeWgWaves * 64),
                     0, stream, (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,
                     (uint16_t*)out, ws_o, ws_lse, Hq, Hkv, S, max_splits, n_hc, total_waves,
                     scale * kLog2e);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || max_splits <= 1) return e;
  hipLaunchKernelGGL((decode_merge_kernel<Tr, D>), dim3((unsigned)(N * Hq)), dim3(64), 0, stream,
                     nullptr, S, ws_o, ws_lse, out, Hq, max_splits, kPagesPerWave);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// float32-query decode: contiguous or paged float32 cache, or paged FP8 e4m3
// cache (VALU).
//
// The reference instantiates its decode and paged kernels for float
// (async_flash_decode_instantiations.cu:4, paged_attention_instantiations.cu)
// and its FP8 paged kernel for float queries and output
// (fp8_paged_attention_instantiations.cu:4, dispatched for at::kFloat at
// fused_softmax_binding.cpp:683-691). fp32 has no 16-bit MFMA operand form
// and decode is HBM-bound, so here the dot products are fp32 FMAs. Per step
// of 64 tokens each lane owns one token for S = q.k (the wave's G query heads
// are broadcast from LDS, pre-scaled to log2 units), the step's max is a
// wave reduction, and for O += P V each lane owns D/64 head-dim elements with
// P broadcast from LDS. FP8 caches decode e4m3 codes exactly to fp32 and fold
// the scales as the reference does (fp8_paged_attention_kernel.cuh:94,104,
// 137): logit = (sum q * code_k) * k_scale, o += p * v_scale * code_v, with
// the scale of the token's physical page (per_block) or of the kv head. Same
// split-K partition (kPagesPerWave pages per wave, split index outermost),
// workspace layout and merge as the 16-bit kernels. A paged sequence's tokens
// past its length are never read into O (their bytes may be anything); block
// ids outside [0, num_blocks) are clamped, as in the 16-bit kernels.
// ---------------------------------------------------------------------------
enum : int { kSrcF32Contig = 0, kSrcF32Paged = 1, kSrcFp8Paged = 2 };

__device__ __forceinline__ float wave_max_f(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = __builtin_fmaxf(x, __shfl_xor(x, off, 64));
  return x;
}
__device__ __forceinline__ float wave_sum_f(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}
// one e4m3 code (byte `b` of w) -> float, exact
__device__ __forceinline__ float e4m3_to_f32(uint32_t w, int b) {
  const f32x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, false);
  const f32x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, true);
  return b == 0 ? lo[0] : b == 1 ? lo[1] : b == 2 ? hi[0] : hi[1];
}

template <int D, int SRC, int G>
__global__ __launch_bounds__(64) void decode_f32_kernel(
    const float* __restrict__ Q, const void* __restrict__ Kc, const void* __restrict__ Vc,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale, int per_block,
    const int32_t* __restrict__ block_tables, const int32_t* __restrict__ context_lens,
    float* __restrict__ O, float* __restrict__ ws_o, float* __restrict__ ws_lse, int Hq,
    int Hkv, int S_contig, int max_blocks, int num_blocks, int max_splits, int n_hc,
    float scale_log2) {
  constexpr bool PAGED = SRC != kSrcF32Contig;
  constexpr bool FP8 = SRC == kSrcFp8Paged;
  constexpr int PER = D / 64;
  constexpr int kSplitTokens = kPagesPerWave * kDecodePage;
  __shared__ float qs[G][D];
  __shared__ float ps[G][64];

  const int lane = threadIdx.x;
  int w = blockIdx.x;
  const int per_split = (int)(gridDim.x / max_splits);
  const int split = w / per_split;
  w %= per_split;
  const int hc = w % n_hc;
  w /= n_hc;
  const int hk = w % Hkv;
  const int n = w / Hkv;
  const int Gq = Hq / Hkv;
  const int hq0 = hk * Gq + hc * G;
  const int Gc = min(G, Gq - hc * G);
  const int L = PAGED ? min(max(0, context_lens[n]), max_blocks * kDecodePage) : S_contig;
  const int n_splits = max(1, (L + kSplitTokens - 1) / kSplitTokens);
  if (split >= n_splits) return;
  const int t_begin = split * kSplitTokens;
  const int t_end = min(t_begin + kSplitTokens, L);

  for (int i = lane; i < G * D; i += 64) {
    const int g = i / D, d = i % D;
    qs[g][d] = (g < Gc) ? Q[((size_t)n * Hq + hq0 + g) * D + d] * scale_log2 : 0.f;
  }
  __syncthreads();

  float m_run[G], l_run[G], o[G][PER];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = kNegInf;
    l_run[g] = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) o[g][i] = 0.f;
  }
  const float* Kf = (const float*)Kc;
  const float* Vf = (const float*)Vc;
  const uint8_t* K8 = (const uint8_t*)Kc;
  const uint8_t* V8 = (const uint8_t*)Vc;
  const float* Kh = PAGED ? Kf : Kf + ((size_t)n * Hkv + hk) * S_contig * D;
  const float* Vh = PAGED ? Vf : Vf + ((size_t)n * Hkv + hk) * S_contig * D;
  const int32_t* bt = PAGED ? block_tables + (size_t)n * max_blocks : nullptr;
  auto block_of = [&](int page) CA_INLINE { return min(max(bt[page], 0), num_blocks - 1); };
  auto kscale_of = [&](int blk) CA_INLINE {
    return per_block ? k_scale[(size_t)blk * Hkv + hk] : k_scale[hk];
  };
  auto vscale_of = [&](int blk) CA_INLINE {
    return per_block ? v_scale[(size_t)blk * Hkv + hk] : v_scale[hk];
  };

  for (int t0 = t_begin; t0 < t_end; t0 += 64) {  // t0 is a multiple of 64: 4 whole pages
    const int t = t0 + lane;
    const bool valid = t < t_end;
    const int tc = valid ? t : t_end - 1;
    float s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) s[g] = 0.f;
    if (FP8) {
      const int blk = block_of(tc / kDecodePage);
      const uint8_t* kp = K8 + ((size_t)blk * Hkv + hk) * D * kDecodePage + (tc % kDecodePage);
#pragma unroll 8
      for (int d = 0; d < D; ++d) {
        const float kv = e4m3_to_f32(kp[d * kDecodePage], 0);
#pragma unroll
        for (int g = 0; g < G; ++g) s[g] = __builtin_fmaf(qs[g][d], kv, s[g]);
      }
      const float ks = kscale_of(blk);
#pragma unroll
      for (int g = 0; g < G; ++g) s[g] *= ks;
    } else if (PAGED) {
      const int blk = block_of(tc / kDecodePage);
      const float* kp = Kf + ((size_t)blk * Hkv + hk) * D * kDecodePage + (tc % kDecodePage);
#pragma unroll 8
      for (int d = 0; d < D; ++d) {
        const float kv = kp[d * kDecodePage];
#pragma unroll
        for (int g = 0; g < G; ++g) s[g] = __builtin_fmaf(qs[g][d], kv, s[g]);
      }
    } else {
      const float* kp = Kh + (size_t)tc * D;
#pragma unroll 4
      for (int d = 0; d < D; d += 4) {
        const float4 kv = *(const float4*)(kp + d);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          s[g] = __builtin_fmaf(qs[g][d], kv.x, s[g]);
          s[g] = __builtin_fmaf(qs[g][d + 1], kv.y, s[g]);
          s[g] = __builtin_fmaf(qs[g][d + 2], kv.z, s[g]);
          s[g] = __builtin_fmaf(qs[g][d + 3], kv.w, s[g]);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float sm = valid ? s[g] : kNegInf;
      const float m_new = __builtin_fmaxf(m_run[g], wave_max_f(sm));
      const float alpha = (m_run[g] == kNegInf) ? 0.f : fast_exp2(m_run[g] - m_new);
      const float p = valid ? fast_exp2(sm - m_new) : 0.f;
      l_run[g] = l_run[g] * alpha + p;
#pragma unroll
      for (int i = 0; i < PER; ++i) o[g][i] *= alpha;
      m_run[g] = m_new;
      ps[g][lane] = p;
    }
    __syncthreads();
    const int nv = min(64, t_end - t0);
    if (PAGED) {
      for (int pg = 0; pg < 4 && 16 * pg < nv; ++pg) {
        const int blk = block_of(t0 / kDecodePage + pg);
        const int cnt = min(16, nv - 16 * pg);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          float vv[16];
          if (FP8) {
            const uint8_t* vrow = V8 + (((size_t)blk * Hkv + hk) * D + lane + 64 * i) * kDecodePage;
            const uint4 x = *(const uint4*)vrow;
            const uint32_t wd[4] = {x.x, x.y, x.z, x.w};
            const float vs = vscale_of(blk);
#pragma unroll
            for (int j = 0; j < 16; j += 2) {
              const f32x2 f = (j & 2) ? __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(wd[j / 4], 1.0f, true)
                                      : __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(wd[j / 4], 1.0f, false);
              vv[j] = f[0] * vs;
              vv[j + 1] = f[1] * vs;
            }
          } else {
            const float* vrow = Vf + (((size_t)blk * Hkv + hk) * D + lane + 64 * i) * kDecodePage;
#pragma unroll
            for (int j = 0; j < 16; j += 4) {
              const float4 x = *(const float4*)(vrow + j);
              vv[j] = x.x; vv[j + 1] = x.y; vv[j + 2] = x.z; vv[j + 3] = x.w;
            }
          }
          for (int j = 0; j < cnt; ++j) {
#pragma unroll
            for (int g = 0; g < G; ++g) o[g][i] = __builtin_fmaf(ps[g][16 * pg + j], vv[j], o[g][i]);
          }
        }
      }
    } else {
      for (int j = 0; j < nv; ++j) {
        const float* vrow = Vh + (size_t)(t0 + j) * D;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const float vv = vrow[lane + 64 * i];
#pragma unroll
          for (int g = 0; g < G; ++g) o[g][i] = __builtin_fmaf(ps[g][j], vv, o[g][i]);
        }
      }
    }
    __syncthreads();
  }

  const bool single = (n_splits == 1);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (g >= Gc) break;
    const float lt = wave_sum_f(l_run[g]);
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const int hq = hq0 + g;
    if (single) {
#pragma unroll
      for (int i = 0; i < PER; ++i) O[((size_t)n * Hq + hq) * D + lane + 64 * i] = o[g][i] * inv;
    } else {
      const size_t sl = ((size_t)n * Hq + hq) * max_splits + split;
#pragma unroll
      for (int i = 0; i < PER; ++i) ws_o[sl * D + lane + 64 * i] = o[g][i] * inv;
      if (lane == 0) ws_lse[sl] = (lt > 0.f) ? m_run[g] + __log2f(lt) : kNegInf;
    }
  }
}

// Arguments of a float32-query decode launch.
struct F32DecodeArgs {
  const void* q;
  const void* kc;
  const void* vc;
  const float* k_scale;
  const float* v_scale;
  int per_block;
  const int32_t* bt;
  const int32_t* lens;
  void* out;
  int N, Hq, Hkv, max_blocks, num_blocks, S_contig;
  float scale;
  void* ws;
  size_t ws_bytes;
};

template <int D, int SRC, int G>
static hipError_t launch_decode_f32_t(const F32DecodeArgs& a, hipStream_t stream) {
  constexpr bool PAGED = SRC != kSrcF32Contig;
  const int max_tokens = PAGED ? a.max_blocks * kDecodePage : a.S_contig;
  const int pages = (max_tokens + kDecodePage - 1) / kDecodePage;
  const int max_splits = max(1, (pages + kPagesPerWave - 1) / kPagesPerWave);
  const int Gq = a.Hq / a.Hkv;
  const int n_hc = (Gq + G - 1) / G;
  const size_t need = decode_workspace_bytes(a.N, a.Hq, D, max_tokens);
  if (a.ws_bytes < need) return hipErrorInvalidValue;
  float* ws_o = (float*)a.ws;
  float* ws_lse = need ? ws_o + (size_t)a.N * a.Hq * max_splits * D : nullptr;
  const long long grid = (long long)a.N * a.Hkv * n_hc * max_splits;
  if (grid == 0) return hipSuccess;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((decode_f32_kernel<D, SRC, G>), dim3((unsigned)grid), dim3(64), 0, stream,
                     (const float*)a.q, a.kc, a.vc, a.k_scale, a.v_scale, a.per_block, a.bt, a.lens,
                     (float*)a.out, ws_o, ws_lse, a.Hq, a.Hkv, a.S_contig, a.max_blocks,
                     a.num_blocks, max_splits, n_hc, a.scale * kLog2e);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || max_splits <= 1) return e;
  hipLaunchKernelGGL((decode_merge_kernel<F32, D>), dim3((unsigned)(a.N * a.Hq)), dim3(64), 0,
                     stream, PAGED ? a.lens : nullptr, max_tokens, ws_o, ws_lse, a.out, a.Hq,
                     max_splits, kPagesPerWave);
  return hipGetLastError();
}

// Query heads per wave for the fp32 kernel: the group size rounded up to a
// power of two, at most 8 (larger groups take several waves).
template <int SRC>
static hipError_t launch_decode_f32(int D, const F32DecodeArgs& a, hipStream_t stream) {
  const int Gq = a.Hq / a.Hkv;
#define CA_F32D(DD, GG) return launch_decode_f32_t<DD, SRC, GG>(a, stream);
#define CA_F32G(DD)                  \
  if (Gq <= 1) { CA_F32D(DD, 1) }    \
  if (Gq <= 2) { CA_F32D(DD, 2) }    \
  if (Gq <= 4) { CA_F32D(DD, 4) }    \
  CA_F32D(DD, 8)
  if (D == 64) { CA_F32G(64) }
  if (D == 128) { CA_F32G(128) }
#undef CA_F32G
#undef CA_F32D
  return hipErrorInvalidValue;
}

hipError_t launch_paged_decode(int dtype, int cache_kind, const void* q, const void* kc,
                               const void* vc, const float* k_scale, const float* v_scale,
                               int per_block_scales, const int32_t* block_tables,
                               const int32_t* context_lens, void* out, int N, int Hq, int Hkv,
                               int D, int max_blocks_per_seq, int num_blocks, float scale,
                               void* ws, size_t ws_bytes, hipStream_t stream) {
#define CA_DEC(TR, DD, KIND)                                                                 \
  if (D == DD)                                                                               \
    return launch_paged_decode_t<TR, DD, KIND>(q, kc, vc, k_scale, v_scale, per_block_scales, \
                                               block_tables, context_lens, out, N, Hq, Hkv,   \
                                               max_blocks_per_seq, num_blocks, scale, ws,      \
                                               ws_bytes, stream);
  if (dtype == kDtypeF32) {
    const F32DecodeArgs a{q,   kc, vc, k_scale, v_scale, per_block_scales, block_tables, context_lens,
                          out, N,  Hq, Hkv,     max_blocks_per_seq, num_blocks, 0, scale, ws, ws_bytes};
    return cache_kind == 0 ? launch_decode_f32<kSrcF32Paged>(D, a, stream)
                           : launch_decode_f32<kSrcFp8Paged>(D, a, stream);
  }
  if (cache_kind == 0) {
    if (dtype == kDtypeBF16) { CA_DEC(BF16, 64, kKindPaged16) CA_DEC(BF16, 128, kKindPaged16) }
    if (dtype == kDtypeF16) { CA_DEC(F16, 64, kKindPaged16) CA_DEC(F16, 128, kKindPaged16) }
  } else {
    if (dtype == kDtypeBF16) { CA_DEC(BF16, 64, kKindPagedFp8) CA_DEC(BF16, 128, kKindPagedFp8) }
    if (dtype == kDtypeF16) { CA_DEC(F16, 64, kKindPagedFp8) CA_DEC(F16, 128, kKindPagedFp8) }
  }
#undef CA_DEC
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// Scratch for the allocation-free FP8 paged decode entry point: the split-K
// partials live in this file-scope device array instead of a caller
// workspace. Each device holds its own copy (at its own address) from the
// library's load until the process ends. Its contents need no clearing: the
// merge reads only the partials its own launch wrote. Calls on one device are
// serialised on it: each call's stream waits for the previous call's launches
// when that call used another stream (an event per device, recorded after
// every launch); under stream capture that ordering is the caller's, as for
// any graph.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
struct ScratchState {
  void* ptr = nullptr;          // device address of `scratch` on this device
  hipEvent_t done = nullptr;    // recorded after the last call's launches
  hipStream_t last = nullptr;   // that call's stream
  bool recorded = false;
};
std::mutex g_scratch_mu;
ScratchState g_scratch[64];
}  // namespace

hipError_t with_noalloc_scratch(hipStream_t stream, const std::function<hipError_t(void*)>& run) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchState& st = g_scratch[dev];
  if (!st.ptr) {
    // set-up, once per device with it current: host code names `scratch`
    // only here (its device address comes from the runtime), and the
    // serialising event is created
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    e = hipEventCreateWithFlags(&st.done, hipEventDisableTiming);
    if (e != hipSuccess) return e;
    st.ptr = p;
  }
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(stream, &cs);
  if (e != hipSuccess) return e;
  const bool capturing = cs != hipStreamCaptureStatusNone;
  if (!capturing && st.recorded && st.last != stream) {
    e = hipStreamWaitEvent(stream, st.done, 0);
    if (e != hipSuccess) return e;
  }
  e = run(st.ptr);
  if (e == hipSuccess && !capturing) {
    e = hipEventRecord(st.done, stream);
    st.last = stream;
    st.recorded = e == hipSuccess;
  }
  return e;
}

size_t paged_decode_partials_bytes(int dtype, int cache_kind, int N, int Hq, int Hkv, int D,
                                   int max_blocks_per_seq) {
  if (dtype == kDtypeF32)
    return split_partials_bytes(N, Hq, D, max_blocks_per_seq / kPagesPerWave +
                                              (max_blocks_per_seq % kPagesPerWave != 0));
#define CA_PLAN(TR, DD, KIND) \
  if (D == DD) return paged_plan<TR, DD, KIND>(N, Hq, Hkv, max_blocks_per_seq).bytes;
  if (cache_kind == 0) {
    if (dtype == kDtypeBF16) { CA_PLAN(BF16, 64, kKindPaged16) CA_PLAN(BF16, 128, kKindPaged16) }
    if (dtype == kDtypeF16) { CA_PLAN(F16, 64, kKindPaged16) CA_PLAN(F16, 128, kKindPaged16) }
  } else {
    if (dtype == kDtypeBF16) { CA_PLAN(BF16, 64, kKindPagedFp8) CA_PLAN(BF16, 128, kKindPagedFp8) }
    if (dtype == kDtypeF16) { CA_PLAN(F16, 64, kKindPagedFp8) CA_PLAN(F16, 128, kKindPagedFp8) }
  }
#undef CA_PLAN
  return 0;
}

hipError_t launch_flash_decode(int dtype, const void* q, const void* k, const void* v, void* o,
                               int B, int Hq, int Hkv, int S, int D, float scale, void* ws,
                               size_t ws_bytes, hipStream_t stream) {
#define CA_FD(TR, DD) \
  if (D == DD) return launch_contig_decode_t<TR, DD>(q, k, v, o, B, Hq, Hkv, S, scale, ws, ws_bytes, stream);
  if (dtype == kDtypeBF16) { CA_FD(BF16, 64) CA_FD(BF16, 128) }
  if (dtype == kDtypeF16) { CA_FD(F16, 64) CA_FD(F16, 128) }
#undef CA_FD
  if (dtype == kDtypeF32) {
    const F32DecodeArgs a{q, k, v, nullptr, nullptr, 0, nullptr, nullptr, o, B, Hq, Hkv, 0, 1, S,
                          scale, ws, ws_bytes};
    return launch_decode_f32<kSrcF32Contig>(D, a, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace ca
