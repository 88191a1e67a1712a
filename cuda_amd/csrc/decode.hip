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
// combines the splits.
#include "common.h"
#include "launch.h"
#include "lds_dma.h"

namespace ca {

enum : int { kKindPaged16 = 0, kKindPagedFp8 = 1, kKindContig16 = 2 };

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

template <int D, int KIND>
struct DecodeGeom {
  static constexpr int NKS = D / 32;  // S^T k-steps (32 d each)
  static constexpr int NB = D / 16;   // PV output blocks (16 d each)
  // 16-byte chunks per lane of one page: 16-bit [D][16] = D/32, fp8 = D/64;
  // contiguous: the K^T operand itself, NKS x 16 B per page
  static constexpr int KREG = KIND == kKindPaged16 ? D / 32 : KIND == kKindPagedFp8 ? D / 64 : NKS;
  // contiguous V: 16 rows x D of one page as 16-byte chunks per lane
  static constexpr int VROWREG = (16 * D * 2) / (64 * 16);
  // wave-private LDS: paged 16-bit K pages [D][16] with a 64-element gap
  // every 8 rows (conflict-free tr16 reads), fp8 K pages [D][16] bytes,
  // contiguous V rows [32][D + 16]
  static constexpr int kPaged16PageElems = D * 16 + (D / 8) * 64;
  static constexpr int kLdsBytesPerWave = KIND == kKindPaged16 ? 2 * kPaged16PageElems * 2
                                          : KIND == kKindPagedFp8 ? 2 * D * 16
                                                                  : 32 * (D + 16) * 2;
};

// Registers of one step (two pages): K and V as loaded from HBM.
template <int D, int KIND>
struct StepRegs {
  using G = DecodeGeom<D, KIND>;
  u32x4 k[2][G::KREG];
  u32x2 v16[2][KIND == kKindPaged16 ? G::NB : 1];
  uint32_t v8[2][KIND == kKindPagedFp8 ? G::NB : 1];
  u32x4 vrow[2][KIND == kKindContig16 ? G::VROWREG : 1];
};

template <typename Tr, int D, int KIND>
// waves per SIMD: fp8 steps fit 3 (168 VGPRs), 16-bit steps carry twice the
// bytes in flight and fit 2
__global__ __launch_bounds__(kDecodeWgWaves * 64)
__attribute__((amdgpu_waves_per_eu(KIND == kKindPagedFp8 ? 3 : 2, KIND == kKindPagedFp8 ? 3 : 2)))
void decode_split_kernel(
    const uint16_t* __restrict__ Q, const void* __restrict__ Kc, const void* __restrict__ Vc,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale, int per_block,
    const int32_t* __restrict__ block_tables, const int32_t* __restrict__ context_lens,
    uint16_t* __restrict__ O, float* __restrict__ ws_o, float* __restrict__ ws_lse, int Hq,
    int Hkv, int max_blocks, int num_blocks, int S_contig, int max_splits, int n_hc,
    long long total_waves, float scale_log2) {
  using vec8 = typename Tr::vec8;
  using vec4 = typename Tr::vec4;
  using vec2 = typename Tr::vec2;
  using G = DecodeGeom<D, KIND>;
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

  // a context longer than its block-table row is cut to the row (never read
  // past block_tables[n][max_blocks - 1])
  const int Lctx = (KIND == kKindContig16) ? S_contig
                                           : min(max(0, context_lens[n]), max_blocks * kDecodePage);
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

  // ---- page ids and per-page scales: lane j < kPagesPerWave holds page p_begin + j ----
  int pid_lane = 0;
  float ksc_lane = 1.f, vsc_lane = 1.f;
  if (KIND != kKindContig16) {
    if (lane < kPagesPerWave && p_begin + lane < p_end) {
      pid_lane = block_tables[(size_t)n * max_blocks + p_begin + lane];
      pid_lane = min(max(pid_lane, 0), num_blocks - 1);
    }
    if (KIND == kKindPagedFp8) {
      if (per_block) {
        if (lane < kPagesPerWave && p_begin + lane < p_end) {
          ksc_lane = k_scale[(size_t)pid_lane * Hkv + hk];
          vsc_lane = v_scale[(size_t)pid_lane * Hkv + hk];
        }
      } else {
        ksc_lane = k_scale[hk];
        vsc_lane = v_scale[hk];
      }
    }
  }
  unsigned char* wlds = lds + wave * G::kLdsBytesPerWave;

  // ---- HBM -> registers for one step ----
  const size_t chunk_elems = (size_t)D * 16;  // one (page, head) chunk
  auto load_step = [&](StepRegs<D, KIND>& R, int step) {
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      const int page = p_begin + 2 * step + pp;
      const bool valid = page < p_end;
      if (KIND == kKindContig16) {
        const size_t base = ((size_t)n * Hkv + hk) * (size_t)S_contig * D;
        const uint16_t* Kp = (const uint16_t*)Kc + base;
        const uint16_t* Vp = (const uint16_t*)Vc + base;
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
      } else {
        const int pid = __builtin_amdgcn_readlane(pid_lane, 2 * step + pp);
        const size_t chunk = ((size_t)pid * Hkv + hk) * chunk_elems;
        if (KIND == kKindPaged16) {
          const uint16_t* Kp = (const uint16_t*)Kc + chunk;
          const uint16_t* Vp = (const uint16_t*)Vc + chunk;
#pragma unroll
          for (int i = 0; i < G::KREG; ++i)
            R.k[pp][i] = valid ? ld_stream<u32x4>(Kp + (lane + 64 * i) * 8) : u32x4{0, 0, 0, 0};
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            R.v16[pp][nb] = valid ? ld_stream<u32x2>(Vp + (16 * nb + l16) * 16 + 4 * grp) : u32x2{0, 0};
        } else {
          const unsigned char* Kp = (const unsigned char*)Kc + chunk;
          const unsigned char* Vp = (const unsigned char*)Vc + chunk;
#pragma unroll
          for (int i = 0; i < G::KREG; ++i)
            R.k[pp][i] = valid ? ld_stream<u32x4>(Kp + (lane + 64 * i) * 16) : u32x4{0, 0, 0, 0};
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            R.v8[pp][nb] = valid ? ld_stream<uint32_t>(Vp + (16 * nb + l16) * 16 + 4 * grp) : 0u;
        }
      }
    }
  };

  f32x4 o[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf, l_run = 0.f;

  // ---- one step of attention on registers R ----
  auto compute_step = [&](const StepRegs<D, KIND>& R, int step) {
    // stage K (paged) or V rows (contiguous) into the wave's LDS
    if (KIND == kKindPaged16) {
      uint16_t* kl = (uint16_t*)wlds;
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
#pragma unroll
        for (int i = 0; i < G::KREG; ++i) {
          const int e = (lane + 64 * i) * 8;  // element offset in the [D][16] page
          *(u32x4*)(kl + pp * G::kPaged16PageElems + e + (e >> 7) * 64) = R.k[pp][i];
        }
    } else if (KIND == kKindPagedFp8) {
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
#pragma unroll
        for (int i = 0; i < G::KREG; ++i)
          *(u32x4*)(wlds + pp * D * 16 + (lane + 64 * i) * 16) = R.k[pp][i];
    } else {
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
      for (int ks = 0; ks < NKS; ++ks) {
        vec8 a;
        if (KIND == kKindPaged16) {
          // tr16: source lane (j = l16/4, c = l16%4) -> row 32ks + 8grp + 4r + j, col 4c
          const uint16_t* kl = (const uint16_t*)wlds + pp * G::kPaged16PageElems;
          const int row = 32 * ks + 8 * grp + (l16 >> 2);
          const int row4 = row + 4;
          const vec4 lo = Tr::tr_read((const CA_LDS void*)(kl + row * 16 + (row >> 3) * 64 + 4 * (l16 & 3)));
          const vec4 hi = Tr::tr_read((const CA_LDS void*)(kl + row4 * 16 + (row4 >> 3) * 64 + 4 * (l16 & 3)));
          a = cat4<vec8, vec4>(lo, hi);
        } else if (KIND == kKindPagedFp8) {
          // tr8: source lane (j = l16/2, c = l16%2) -> row 32ks + 8grp + j, col 8c
          const int row = 32 * ks + 8 * grp + (l16 >> 1);
          const i32x2 raw = tr8_read((const CA_LDS void*)(wlds + pp * D * 16 + row * 16 + 8 * (l16 & 1)));
          a = fp8x8_to<Tr>((uint32_t)raw[0], (uint32_t)raw[1]);
        } else {
          a = __builtin_bit_cast(vec8, R.k[pp][ks]);
        }
        s[pp] = Tr::mfma16(a, qv[ks], s[pp]);
      }
    }

    // online softmax over the step's 32 tokens
    const int pageA = p_begin + 2 * step;
    float cA = scale_log2, cB = scale_log2, vsA = 1.f, vsB = 1.f;
    if (KIND == kKindPagedFp8) {
      cA *= __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ksc_lane), 2 * step));
      cB *= __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ksc_lane), 2 * step + 1));
      vsA = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(vsc_lane), 2 * step));
      vsB = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(vsc_lane), 2 * step + 1));
    }
    float x[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = s[0][r] * cA;
      x[4 + r] = s[1][r] * cB;
    }
    // tokens past the context (or the wave's last page) are masked; their V
    // slots are zeroed too, so stale cache bytes (NaN patterns included) in
    // a partially filled page cannot reach the PV product
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
      const vec2 ua = Tr::pack2(p[2 * j] * vsA, p[2 * j + 1] * vsA);
      const vec2 ub = Tr::pack2(p[4 + 2 * j] * vsB, p[4 + 2 * j + 1] * vsB);
      pa[2 * j] = ua[0];
      pa[2 * j + 1] = ua[1];
      pa[4 + 2 * j] = ub[0];
      pa[4 + 2 * j + 1] = ub[1];
    }

    // O += P V^T
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      vec8 bv;
      if (KIND == kKindPaged16) {
        bv = cat4<vec8, vec4>(__builtin_bit_cast(vec4, R.v16[0][nb]), __builtin_bit_cast(vec4, R.v16[1][nb]));
      } else if (KIND == kKindPagedFp8) {
        bv = fp8x8_to<Tr>(R.v8[0][nb], R.v8[1][nb]);
      } else {
        // tr16: source lane (j = l16/4, c = l16%4) -> row (16pp + 4grp + j), col 16nb + 4c
        const uint16_t* vl = (const uint16_t*)wlds;
        const int row = 4 * grp + (l16 >> 2);
        const int col = 16 * nb + 4 * (l16 & 3);
        const vec4 lo = Tr::tr_read((const CA_LDS void*)(vl + row * (D + 16) + col));
        const vec4 hi = Tr::tr_read((const CA_LDS void*)(vl + (16 + row) * (D + 16) + col));
        bv = cat4<vec8, vec4>(lo, hi);
      }
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
  StepRegs<D, KIND> A, B;
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
// V pages linear [D][16].
// ---------------------------------------------------------------------------
#ifndef CA_DEC_SPLIT_OUTER
#define CA_DEC_SPLIT_OUTER 2
#endif
// Cache policy of the page loads: "nt" (every byte is read once per launch,
// so it is streamed rather than retained).
#ifndef CA_DMA_POLICY
#define CA_DMA_POLICY 2
#endif

#ifndef CA_DMA_PPS
#define CA_DMA_PPS 1
#endif
#ifndef CA_RING_FP8
#define CA_RING_FP8 4
#endif
#ifndef CA_RING_16
#define CA_RING_16 3
#endif
// Pages per split of the direct-load decode (64 or 128: one or two page-id
// registers per lane): 256 KB of K and V per split for both cache kinds
// (128 fp8 pages, 64 16-bit pages). A split's start (context length,
// block-table row, scales, filling the ring) is paid once per split: 128
// fp8 pages measured +3.5 % on C4 over 64, while 128 16-bit pages leave C3
// too few waves (-3 %).
#ifndef CA_DMA_PAGES_FP8
#define CA_DMA_PAGES_FP8 128
#endif
// Pages per step and ring depth of the direct-load decode. One page per step
// keeps a ring slot small (K + V of one page), so more waves fit a CU's LDS
// and more bytes are in flight per CU; the PV product then runs on 16x16x16
// MFMAs, whose 4 k-values per lane are exactly the 4 tokens a lane holds.
template <int KIND>
struct DmaCfg {
  static constexpr int kPagesPerStep = CA_DMA_PPS;
  static constexpr int kRing = KIND == kKindPagedFp8 ? CA_RING_FP8 : CA_RING_16;
  static constexpr int kPages = KIND == kKindPagedFp8 ? CA_DMA_PAGES_FP8 : kPagesPerWave;
  // decode_workspace_bytes sizes the partials for kPagesPerWave-page splits
  static_assert(kPages >= kPagesPerWave, "pages per split");
};

template <typename Tr, int D, int KIND>
__global__ __launch_bounds__(64) void decode_dma_kernel(
    const uint16_t* __restrict__ Q, const void* __restrict__ Kc, const void* __restrict__ Vc,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale, int per_block,
    const int32_t* __restrict__ block_tables, const int32_t* __restrict__ context_lens,
    uint16_t* __restrict__ O, float* __restrict__ ws_o, float* __restrict__ ws_lse, int Hq,
    int Hkv, int max_blocks, int num_blocks, int max_splits, int n_hc, float scale_log2) {
  using vec8 = typename Tr::vec8;
  using vec4 = typename Tr::vec4;
  using vec2 = typename Tr::vec2;
  constexpr int NKS = D / 32, NB = D / 16;
  constexpr bool FP8 = KIND == kKindPagedFp8;
  constexpr int ELEM = FP8 ? 1 : 2;
  constexpr int CHUNK = D * 16 * ELEM;        // bytes of one (page, head) chunk
  constexpr int NDMA = CHUNK / 1024;          // 16 B x 64 lanes per load
  constexpr int PPS = DmaCfg<KIND>::kPagesPerStep;
  constexpr int STAGE = 2 * PPS * CHUNK;      // K and V of the step's pages
  constexpr int RING = DmaCfg<KIND>::kRing;
  constexpr int DPS = 2 * PPS * NDMA;         // loads per step
  constexpr int KRD = FP8 ? NKS : 2 * NKS;    // LDS reads for one page's K^T operands
  static_assert(PPS == 1 || PPS == 2, "pages per step");
  constexpr int kDmaPages = DmaCfg<KIND>::kPages;
  constexpr int PB = kDmaPages / 64;          // page-id registers per lane
  static_assert(kDmaPages % 64 == 0 && PB <= 2, "pages per split");
  static_assert((RING - 1) * DPS <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) unsigned char ring[RING * STAGE];

  const int lane = threadIdx.x;
  int w = blockIdx.x;
#if CA_DEC_SPLIT_OUTER == 2
  // split index outermost, counted from each sequence's end: the waves of
  // splits before a sequence's start (none exist) come first and retire at
  // once, and every sequence's last (partial) split is in the final group
  const int per_split = (int)(gridDim.x / max_splits);
  const int from_end = max_splits - 1 - w / per_split;
  w %= per_split;
#elif CA_DEC_SPLIT_OUTER
  // split index outermost: every sequence's first splits come first and the
  // waves of splits past a sequence's end gather at the tail of the grid
  const int per_split = (int)(gridDim.x / max_splits);
  const int split = w / per_split;
  w %= per_split;
#else
  const int split = w % max_splits;
  w /= max_splits;
#endif
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
#if CA_DEC_SPLIT_OUTER == 2
  const int split = n_splits - 1 - from_end;
  if (split < 0) return;
#else
  if (split >= n_splits) return;
#endif

  const int l16 = lane & 15, grp = lane >> 4;
  const int p_begin = split * kDmaPages;
  const int p_end = min(p_begin + kDmaPages, n_pages);
  const int n_steps = (p_end - p_begin + PPS - 1) / PPS;

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
      pid_lane[pb] = block_tables[(size_t)n * max_blocks + page];
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
  const unsigned char* dummy = (const unsigned char*)Q;  // 16 valid bytes for padding loads
  auto issue_step = [&](int step, int slot) {
    unsigned char* base = ring + slot * STAGE;
#pragma unroll
    for (int pp = 0; pp < PPS; ++pp) {
      const int page = p_begin + PPS * step + pp;
      const bool valid = step < n_steps && page < p_end;
      const int idx = valid ? PPS * step + pp : 0;
      const int pid = lane_val(pid_lane, idx);
      const size_t chunk = ((size_t)pid * Hkv + hk) * (size_t)CHUNK;
      const unsigned char* kp = (const unsigned char*)Kc + chunk;
      const unsigned char* vp = (const unsigned char*)Vc + chunk;
#pragma unroll
      for (int i = 0; i < NDMA; ++i) {
        dma16<CA_DMA_POLICY>(valid ? kp + k_src(i) : dummy, (CA_LDS void*)(base + pp * 2 * CHUNK + 1024 * i));
        dma16<CA_DMA_POLICY>(valid ? vp + 1024 * i + 16 * lane : dummy,
              (CA_LDS void*)(base + pp * 2 * CHUNK + CHUNK + 1024 * i));
      }
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
  const uint32_t v_off = (uint32_t)(16 * l16 + 4 * grp) * ELEM;
  const uint32_t ring0 = lds_off(ring);

  f32x4 o[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf, l_run = 0.f;

#pragma unroll
  // RING steps in flight from the start; a slot is refilled as soon as its
  // LDS reads have returned, so RING steps stay in flight during the math
  for (int s = 0; s < RING; ++s) issue_step(s, s);
  int slot = 0;
  for (int step = 0; step < n_steps; ++step) {
    wait_vmcnt<(RING - 1) * DPS>();  // this step's loads are the oldest outstanding
    const uint32_t sb = ring0 + slot * STAGE;

    // ---- LDS -> operands ----
    u32x2 kraw[PPS][KRD];
    uint32_t v8r[PPS][FP8 ? NB : 1];
    u32x2 v16r[PPS][FP8 ? 1 : NB];
#pragma unroll
    for (int pp = 0; pp < PPS; ++pp) {
      const uint32_t kb = sb + pp * 2 * CHUNK;
      const uint32_t vb = kb + CHUNK + v_off;
      if (FP8) {
        const uint32_t a = kb + k_lo;
        kraw[pp][0] = lds_read_tr8<0>(a);
        if (NKS > 1) kraw[pp][1 % KRD] = lds_read_tr8<512>(a);
        if (NKS > 2) kraw[pp][2 % KRD] = lds_read_tr8<1024>(a);
        if (NKS > 3) kraw[pp][3 % KRD] = lds_read_tr8<1536>(a);
#define CA_V8(NBI) if (NBI < NB) v8r[pp][NBI % NB] = lds_read_b32<256 * NBI>(vb);
        CA_V8(0) CA_V8(1) CA_V8(2) CA_V8(3) CA_V8(4) CA_V8(5) CA_V8(6) CA_V8(7)
#undef CA_V8
      } else {
        const uint32_t alo = kb + k_lo, ahi = kb + k_hi;
        kraw[pp][0] = lds_read_tr16<0>(alo);
        kraw[pp][1] = lds_read_tr16<0>(ahi);
        if (NKS > 1) { kraw[pp][2 % KRD] = lds_read_tr16<1024>(alo); kraw[pp][3 % KRD] = lds_read_tr16<1024>(ahi); }
        if (NKS > 2) { kraw[pp][4 % KRD] = lds_read_tr16<2048>(alo); kraw[pp][5 % KRD] = lds_read_tr16<2048>(ahi); }
        if (NKS > 3) { kraw[pp][6 % KRD] = lds_read_tr16<3072>(alo); kraw[pp][7 % KRD] = lds_read_tr16<3072>(ahi); }
#define CA_V16(NBI) if (NBI < NB) v16r[pp][NBI % NB] = lds_read_b64<512 * NBI>(vb);
        CA_V16(0) CA_V16(1) CA_V16(2) CA_V16(3) CA_V16(4) CA_V16(5) CA_V16(6) CA_V16(7)
#undef CA_V16
      }
    }
    wait_lgkm0();
#pragma unroll
    for (int pp = 0; pp < PPS; ++pp) {
#pragma unroll
      for (int i = 0; i < KRD; ++i) after_wait(kraw[pp][i]);
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        if (FP8) after_wait(v8r[pp][i % (FP8 ? NB : 1)]);
        else after_wait(v16r[pp][i % (FP8 ? 1 : NB)]);
      }
    }
    issue_step(step + RING, slot);  // the slot's data is in registers now

    // ---- S^T per page ----
    f32x4 s[PPS];
#pragma unroll
    for (int pp = 0; pp < PPS; ++pp) {
      s[pp] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        vec8 a;
        if (FP8) {
          a = fp8x8_to<Tr>(kraw[pp][ks % KRD][0], kraw[pp][ks % KRD][1]);
        } else {
          const u32x4 t = {kraw[pp][(2 * ks) % KRD][0], kraw[pp][(2 * ks) % KRD][1],
                           kraw[pp][(2 * ks + 1) % KRD][0], kraw[pp][(2 * ks + 1) % KRD][1]};
          a = __builtin_bit_cast(vec8, t);
        }
        s[pp] = Tr::mfma16(a, qv[ks], s[pp]);
      }
    }

    // ---- online softmax over the step's 16 * PPS tokens ----
    const int page0 = p_begin + PPS * step;
    float c[PPS], vs[PPS];
#pragma unroll
    for (int pp = 0; pp < PPS; ++pp) {
      c[pp] = scale_log2;
      vs[pp] = 1.f;
      if (FP8) {
        c[pp] *= lane_val(ksc_lane, PPS * step + pp);
        vs[pp] = lane_val(vsc_lane, PPS * step + pp);
      }
    }
    float x[4 * PPS];
#pragma unroll
    for (int pp = 0; pp < PPS; ++pp)
#pragma unroll
      for (int r = 0; r < 4; ++r) x[4 * pp + r] = s[pp][r] * c[pp];
    // tokens past the context (or the wave's last page) are masked; their V
    // slots are zeroed too, so stale cache bytes (NaN patterns included) in
    // a partially filled page cannot reach the PV product
    const bool partial = (page0 + PPS) * 16 > Lctx || page0 + PPS > p_end;
    bool slot_ok[4 * PPS];
#pragma unroll
    for (int pp = 0; pp < PPS; ++pp)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        slot_ok[4 * pp + r] = ((page0 + pp) * 16 + 4 * grp + r < Lctx) && (page0 + pp < p_end);
    if (partial) {
#pragma unroll
      for (int i = 0; i < 4 * PPS; ++i)
        if (!slot_ok[i]) x[i] = kNegInf;
    }
    float tmax = max3(x[0], x[1], __builtin_fmaxf(x[2], x[3]));
    if (PPS == 2) tmax = max3(tmax, __builtin_fmaxf(x[4 % (4 * PPS)], x[5 % (4 * PPS)]),
                              __builtin_fmaxf(x[6 % (4 * PPS)], x[7 % (4 * PPS)]));
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
    float p[4 * PPS];
#pragma unroll
    for (int i = 0; i < 4 * PPS; ++i) p[i] = fast_exp2(x[i] - msub);
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 4 * PPS; ++i) psum += p[i];
    l_run += psum;
    // P operand (v scale folded in): PPS = 2 -> 8 values = 4 tokens of each
    // page (16x16x32); PPS = 1 -> the lane's 4 tokens (16x16x16)
    u32x4 pw;
#pragma unroll
    for (int pp = 0; pp < PPS; ++pp) {
      pw[2 * pp] = __builtin_bit_cast(uint32_t, Tr::pack2(p[4 * pp] * vs[pp], p[4 * pp + 1] * vs[pp]));
      pw[2 * pp + 1] = __builtin_bit_cast(uint32_t, Tr::pack2(p[4 * pp + 2] * vs[pp], p[4 * pp + 3] * vs[pp]));
    }

    // ---- O += P V^T ----
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      u32x4 bw;
#pragma unroll
      for (int pp = 0; pp < PPS; ++pp) {
        if (FP8) {
          const uint32_t v = v8r[pp][nb % (FP8 ? NB : 1)];
          bw[2 * pp] = __builtin_bit_cast(uint32_t, Fp8Conv<Tr>::template cvt<false>(v));
          bw[2 * pp + 1] = __builtin_bit_cast(uint32_t, Fp8Conv<Tr>::template cvt<true>(v));
        } else {
          bw[2 * pp] = v16r[pp][nb % (FP8 ? 1 : NB)][0];
          bw[2 * pp + 1] = v16r[pp][nb % (FP8 ? 1 : NB)][1];
        }
      }
      if (partial) {
        // zero masked token slots: 16-bit halves of the operand dwords
#pragma unroll
        for (int i = 0; i < 4 * PPS; ++i)
          if (!slot_ok[i]) bw[i >> 1] &= (i & 1) ? 0x0000ffffu : 0xffff0000u;
      }
      if (PPS == 2) {
        o[nb] = Tr::mfma16(__builtin_bit_cast(vec8, pw), __builtin_bit_cast(vec8, bw), o[nb]);
      } else {
        const u32x2 a2 = {pw[0], pw[1]}, b2 = {bw[0], bw[1]};
        o[nb] = Tr::mfma16k16(__builtin_bit_cast(vec4, a2), __builtin_bit_cast(vec4, b2), o[nb]);
      }
    }
    slot = (slot == RING - 1) ? 0 : slot + 1;
  }
  wait_vmcnt<0>();  // no load may still target this workgroup's LDS when it exits

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
      const size_t sl = ((size_t)n * Hq + hq) * max_splits + split;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) ws_o[sl * D + 16 * nb + l16] = o[nb][r] * inv;
      if (l16 == 0) ws_lse[sl] = (lg > 0.f) ? mg + __log2f(lg) : kNegInf;
    }
  }
}

// Combines the split partials of every (sequence, query head) with more than
// one split: o = sum_s 2^(lse_s - M) o_s / sum_s 2^(lse_s - M). One wave per
// (sequence, head); each lane owns D/64 output elements.
template <typename Tr, int D>
__global__ __launch_bounds__(64) void decode_merge_kernel(
    const int32_t* __restrict__ context_lens, int max_tokens, const float* __restrict__ ws_o,
    const float* __restrict__ ws_lse, void* __restrict__ O, int Hq, int max_splits,
    int pages_per_split) {
  constexpr int PER = D / 64;
  const int n = blockIdx.x / Hq, hq = blockIdx.x % Hq;
  const int lane = threadIdx.x;
  const int Lctx = context_lens ? min(max(0, context_lens[n]), max_tokens) : max_tokens;
  const int n_pages = (Lctx + kDecodePage - 1) / kDecodePage;
  const int n_splits = (n_pages + pages_per_split - 1) / pages_per_split;
  if (n_splits <= 1) return;
  const size_t slot0 = ((size_t)n * Hq + hq) * max_splits;
  float M = kNegInf;
  for (int s = lane; s < n_splits; s += 64) M = __builtin_fmaxf(M, ws_lse[slot0 + s]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) M = __builtin_fmaxf(M, __shfl_xor(M, off, 64));
  float wsum = 0.f;
  float acc[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) acc[i] = 0.f;
  if (M != kNegInf) {
    for (int s0 = 0; s0 < n_splits; s0 += 64) {
      const int s = s0 + lane;
      const float lse = (s < n_splits) ? ws_lse[slot0 + s] : kNegInf;
      const float wl = (lse == kNegInf) ? 0.f : fast_exp2(lse - M);
      const int cnt = min(64, n_splits - s0);
#pragma unroll 4
      for (int j = 0; j < cnt; ++j) {
        const float wj = __shfl(wl, j, 64);
        wsum += wj;
        const float* src = ws_o + (slot0 + s0 + j) * D + lane * PER;
#pragma unroll
        for (int i = 0; i < PER; ++i) acc[i] += wj * src[i];
      }
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) Tr::store(O, ((size_t)n * Hq + hq) * D + lane * PER + i, acc[i] * inv);
}

size_t decode_workspace_bytes(int N, int Hq, int D, int max_tokens) {
  const int pages = (max_tokens + kDecodePage - 1) / kDecodePage;
  const int max_splits = (pages + kPagesPerWave - 1) / kPagesPerWave;
  if (max_splits <= 1) return 0;
  return (size_t)N * Hq * max_splits * (size_t)(D + 1) * sizeof(float);
}

template <typename Tr, int D, int KIND>
static hipError_t launch_decode_t(const void* q, const void* kc, const void* vc,
                                  const float* k_scale, const float* v_scale, int per_block,
                                  const int32_t* bt, const int32_t* lens, void* out, int N,
                                  int Hq, int Hkv, int max_blocks, int num_blocks, int S_contig,
                                  float scale, void* ws, size_t ws_bytes, hipStream_t stream) {
  const int max_tokens = (KIND == kKindContig16) ? S_contig : max_blocks * kDecodePage;
  const int pages = (max_tokens + kDecodePage - 1) / kDecodePage;
  // the direct-load kernel splits at DmaCfg<KIND>::kPages pages, the others
  // at kPagesPerWave; the workspace (sized for kPagesPerWave-page splits)
  // covers both
  const bool dma = KIND != kKindContig16 && kDecodeDma;
  const int pps = dma ? DmaCfg<KIND>::kPages : kPagesPerWave;
  const int max_splits = max(1, (pages + pps - 1) / pps);
  const int Gq = Hq / Hkv;
  const int n_hc = (Gq + 15) / 16;
  const size_t need = decode_workspace_bytes(N, Hq, D, max_tokens);
  if (ws_bytes < need) return hipErrorInvalidValue;
  float* ws_o = (float*)ws;
  float* ws_lse = need ? ws_o + (size_t)N * Hq * max_splits * D : nullptr;
  const long long total_waves = (long long)N * Hkv * n_hc * max_splits;
  if (total_waves == 0) return hipSuccess;
  if (dma) {
    if (total_waves > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL((decode_dma_kernel<Tr, D, KIND>), dim3((unsigned)total_waves), dim3(64), 0,
                       stream, (const uint16_t*)q, kc, vc, k_scale, v_scale, per_block, bt, lens,
                       (uint16_t*)out, ws_o, ws_lse, Hq, Hkv, max_blocks, num_blocks, max_splits,
                       n_hc, scale * kLog2e);
  } else {
    const long long grid = (total_waves + kDecodeWgWaves - 1) / kDecodeWgWaves;
    if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL((decode_split_kernel<Tr, D, KIND>), dim3((unsigned)grid),
                       dim3(kDecodeWgWaves * 64), 0, stream, (const uint16_t*)q, kc, vc, k_scale,
                       v_scale, per_block, bt, lens, (uint16_t*)out, ws_o, ws_lse, Hq, Hkv,
                       max_blocks, num_blocks, S_contig, max_splits, n_hc, total_waves,
                       scale * kLog2e);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || max_splits <= 1) return e;
  hipLaunchKernelGGL((decode_merge_kernel<Tr, D>), dim3((unsigned)(N * Hq)), dim3(64), 0, stream,
                     KIND == kKindContig16 ? nullptr : lens, max_tokens, ws_o, ws_lse, out, Hq,
                     max_splits, pps);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// float32 decode, contiguous or paged cache (VALU).
//
// The reference instantiates its decode and paged kernels for float
// (async_flash_decode_instantiations.cu:4, paged_attention_instantiations.cu);
// fp32 has no 16-bit MFMA operand form and decode is HBM-bound, so here the
// dot products are fp32 FMAs. Per step of 64 tokens each lane owns one token
// for S = q.k (the wave's G query heads are broadcast from LDS, pre-scaled to
// log2 units), the step's max is a wave reduction, and for O += P V each lane
// owns D/64 head-dim elements with P broadcast from LDS. Same split-K
// partition (kPagesPerWave pages per wave, split index outermost), workspace
// layout and merge as the 16-bit kernels. A paged sequence's tokens past its
// length are never read into O (their bytes may be anything).
// ---------------------------------------------------------------------------
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

template <int D, bool PAGED, int G>
__global__ __launch_bounds__(64) void decode_f32_kernel(
    const float* __restrict__ Q, const float* __restrict__ Kc, const float* __restrict__ Vc,
    const int32_t* __restrict__ block_tables, const int32_t* __restrict__ context_lens,
    float* __restrict__ O, float* __restrict__ ws_o, float* __restrict__ ws_lse, int Hq,
    int Hkv, int S_contig, int max_blocks, int max_splits, int n_hc, float scale_log2) {
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
  const float* Kh = PAGED ? Kc : Kc + ((size_t)n * Hkv + hk) * S_contig * D;
  const float* Vh = PAGED ? Vc : Vc + ((size_t)n * Hkv + hk) * S_contig * D;
  const int32_t* bt = PAGED ? block_tables + (size_t)n * max_blocks : nullptr;

  for (int t0 = t_begin; t0 < t_end; t0 += 64) {  // t0 is a multiple of 64: 4 whole pages
    const int t = t0 + lane;
    const bool valid = t < t_end;
    const int tc = valid ? t : t_end - 1;
    float s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) s[g] = 0.f;
    if (PAGED) {
      const int blk = bt[tc / kDecodePage];
      const float* kp = Kc + ((size_t)blk * Hkv + hk) * D * kDecodePage + (tc % kDecodePage);
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
        const int blk = bt[t0 / kDecodePage + pg];
        const float* vp = Vc + ((size_t)blk * Hkv + hk) * D * kDecodePage;
        const int cnt = min(16, nv - 16 * pg);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const float* vrow = vp + (size_t)(lane + 64 * i) * kDecodePage;
          float vv[16];
#pragma unroll
          for (int j = 0; j < 16; j += 4) {
            const float4 x = *(const float4*)(vrow + j);
            vv[j] = x.x; vv[j + 1] = x.y; vv[j + 2] = x.z; vv[j + 3] = x.w;
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

template <int D, bool PAGED, int G>
static hipError_t launch_decode_f32_t(const void* q, const void* kc, const void* vc,
                                      const int32_t* bt, const int32_t* lens, void* out, int N,
                                      int Hq, int Hkv, int max_blocks, int S_contig, float scale,
                                      void* ws, size_t ws_bytes, hipStream_t stream) {
  const int max_tokens = PAGED ? max_blocks * kDecodePage : S_contig;
  const int pages = (max_tokens + kDecodePage - 1) / kDecodePage;
  const int max_splits = max(1, (pages + kPagesPerWave - 1) / kPagesPerWave);
  const int Gq = Hq / Hkv;
  const int n_hc = (Gq + G - 1) / G;
  const size_t need = decode_workspace_bytes(N, Hq, D, max_tokens);
  if (ws_bytes < need) return hipErrorInvalidValue;
  float* ws_o = (float*)ws;
  float* ws_lse = need ? ws_o + (size_t)N * Hq * max_splits * D : nullptr;
  const long long grid = (long long)N * Hkv * n_hc * max_splits;
  if (grid == 0) return hipSuccess;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((decode_f32_kernel<D, PAGED, G>), dim3((unsigned)grid), dim3(64), 0, stream,
                     (const float*)q, (const float*)kc, (const float*)vc, bt, lens, (float*)out,
                     ws_o, ws_lse, Hq, Hkv, S_contig, max_blocks, max_splits, n_hc,
                     scale * kLog2e);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || max_splits <= 1) return e;
  hipLaunchKernelGGL((decode_merge_kernel<F32, D>), dim3((unsigned)(N * Hq)), dim3(64), 0, stream,
                     PAGED ? lens : nullptr, max_tokens, ws_o, ws_lse, out, Hq, max_splits,
                     kPagesPerWave);
  return hipGetLastError();
}

// Query heads per wave for the fp32 kernel: the group size rounded up to a
// power of two, at most 8 (larger groups take several waves).
template <int D, bool PAGED>
static hipError_t launch_decode_f32(const void* q, const void* kc, const void* vc,
                                    const int32_t* bt, const int32_t* lens, void* out, int N,
                                    int Hq, int Hkv, int max_blocks, int S_contig, float scale,
                                    void* ws, size_t ws_bytes, hipStream_t stream) {
  const int Gq = Hq / Hkv;
#define CA_F32D(GG)                                                                          \
  return launch_decode_f32_t<D, PAGED, GG>(q, kc, vc, bt, lens, out, N, Hq, Hkv, max_blocks, \
                                           S_contig, scale, ws, ws_bytes, stream);
  if (Gq <= 1) { CA_F32D(1) }
  if (Gq <= 2) { CA_F32D(2) }
  if (Gq <= 4) { CA_F32D(4) }
  CA_F32D(8)
#undef CA_F32D
}

hipError_t launch_paged_decode(int dtype, int cache_kind, const void* q, const void* kc,
                               const void* vc, const float* k_scale, const float* v_scale,
                               int per_block_scales, const int32_t* block_tables,
                               const int32_t* context_lens, void* out, int N, int Hq, int Hkv,
                               int D, int max_blocks_per_seq, int num_blocks, float scale,
                               void* ws, size_t ws_bytes, hipStream_t stream) {
#define CA_DEC(TR, DD, KIND)                                                                \
  if (D == DD)                                                                              \
    return launch_decode_t<TR, DD, KIND>(q, kc, vc, k_scale, v_scale, per_block_scales,     \
                                         block_tables, context_lens, out, N, Hq, Hkv,       \
                                         max_blocks_per_seq, num_blocks, 0, scale, ws,      \
                                         ws_bytes, stream);
  if (cache_kind == 0) {
    if (dtype == kDtypeF32) {
      if (D == 64)
        return launch_decode_f32<64, true>(q, kc, vc, block_tables, context_lens, out, N, Hq, Hkv,
                                           max_blocks_per_seq, 0, scale, ws, ws_bytes, stream);
      if (D == 128)
        return launch_decode_f32<128, true>(q, kc, vc, block_tables, context_lens, out, N, Hq, Hkv,
                                            max_blocks_per_seq, 0, scale, ws, ws_bytes, stream);
    }
    if (dtype == kDtypeBF16) { CA_DEC(BF16, 64, kKindPaged16) CA_DEC(BF16, 128, kKindPaged16) }
    if (dtype == kDtypeF16) { CA_DEC(F16, 64, kKindPaged16) CA_DEC(F16, 128, kKindPaged16) }
  } else {
    if (dtype == kDtypeBF16) { CA_DEC(BF16, 64, kKindPagedFp8) CA_DEC(BF16, 128, kKindPagedFp8) }
    if (dtype == kDtypeF16) { CA_DEC(F16, 64, kKindPagedFp8) CA_DEC(F16, 128, kKindPagedFp8) }
  }
#undef CA_DEC
  return hipErrorInvalidValue;
}

hipError_t launch_flash_decode(int dtype, const void* q, const void* k, const void* v, void* o,
                               int B, int Hq, int Hkv, int S, int D, float scale, void* ws,
                               size_t ws_bytes, hipStream_t stream) {
#define CA_FD(TR, DD)                                                                        \
  if (D == DD)                                                                               \
    return launch_decode_t<TR, DD, kKindContig16>(q, k, v, nullptr, nullptr, 0, nullptr,     \
                                                  nullptr, o, B, Hq, Hkv, 0, 0, S, scale, ws, \
                                                  ws_bytes, stream);
  if (dtype == kDtypeBF16) { CA_FD(BF16, 64) CA_FD(BF16, 128) }
  if (dtype == kDtypeF16) { CA_FD(F16, 64) CA_FD(F16, 128) }
#undef CA_FD
  if (dtype == kDtypeF32) {
    if (D == 64)
      return launch_decode_f32<64, false>(q, k, v, nullptr, nullptr, o, B, Hq, Hkv, 0, S, scale,
                                          ws, ws_bytes, stream);
    if (D == 128)
      return launch_decode_f32<128, false>(q, k, v, nullptr, nullptr, o, B, Hq, Hkv, 0, S, scale,
                                           ws, ws_bytes, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace ca
