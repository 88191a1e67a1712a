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
// Work decomposition (split-K)
//   workgroup = (sequence n, kv head, query-head chunk of <= 16, split);
//   a split covers kPagesPerSplit pages of 16 tokens, 4 waves x 16 pages;
//   each wave walks its pages two at a time with the next two prefetched.
//   The GQA group of query heads (Hq / Hkv <= 16 per chunk) shares every K/V
//   byte loaded, so each cache byte is read from HBM once per kv head.
// Per wave and two pages (16x16x32 MFMAs, query heads padded to 16):
//   S^T[16 tok x 16 heads] = K^T Q^T per page; the page is [D][16] with
//   tokens contiguous, so the K^T operand (8 consecutive d for one token) is
//   read from a wave-private LDS copy with ds_read_b64_tr_b16 / _tr_b8;
//   online softmax over tokens, lazily rescaled;
//   O[16 heads x D] += P V^T over the 32 tokens; the V^T operand (tokens
//   contiguous for one d) comes straight from HBM in operand layout.
//   FP8: codes are converted exactly to the MFMA element type; the k scale of
//   a page multiplies that page's logits and the v scale is folded into P.
// The 4 waves merge through LDS; a sequence with one split writes its output
// directly, otherwise a partial (o / l, log2-sum-exp) goes to the workspace
// and decode_merge_kernel combines the splits.
#include "common.h"
#include "launch.h"

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

template <typename Tr>
__device__ __forceinline__ typename Tr::vec8 fp8x8_to(uint32_t lo, uint32_t hi) {
  using vec2 = typename Tr::vec2;
  using vec8 = typename Tr::vec8;
  const vec2 a = Fp8Conv<Tr>::template cvt<false>(lo), b = Fp8Conv<Tr>::template cvt<true>(lo);
  const vec2 c = Fp8Conv<Tr>::template cvt<false>(hi), d = Fp8Conv<Tr>::template cvt<true>(hi);
  vec8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
  r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
  return r;
}

template <int D, int KIND>
struct DecodeLds {
  // per-wave staging of the two pages of one step
  //   paged 16-bit: K pages [D][16] with a 64-element gap every 8 rows
  //   paged fp8:    K pages [D][16] bytes, no gap
  //   contiguous:   V rows [32][D + 16]
  static constexpr int kPaged16PageElems = D * 16 + (D / 8) * 64;
  static constexpr int kBytesPerWave =
      KIND == kKindPaged16 ? 2 * kPaged16PageElems * 2
      : KIND == kKindPagedFp8 ? 2 * D * 16
                              : 32 * (D + 16) * 2;
  static constexpr int kStageBytes = kDecodeWaves * kBytesPerWave;
  static constexpr int kMergeBytes = kDecodeWaves * 16 * D * 4;
  static constexpr int kBytes = kStageBytes > kMergeBytes ? kStageBytes : kMergeBytes;
};

template <typename Tr, int D, int KIND>
__global__ __launch_bounds__(kDecodeWaves * 64) void decode_split_kernel(
    const uint16_t* __restrict__ Q, const void* __restrict__ Kc, const void* __restrict__ Vc,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale, int per_block,
    const int32_t* __restrict__ block_tables, const int32_t* __restrict__ context_lens,
    uint16_t* __restrict__ O, float* __restrict__ ws_o, float* __restrict__ ws_lse, int Hq,
    int Hkv, int max_blocks, int num_blocks, int S_contig, int max_splits, int n_hc,
    float scale_log2) {
  using vec8 = typename Tr::vec8;
  using vec4 = typename Tr::vec4;
  using vec2 = typename Tr::vec2;
  constexpr int NKS = D / 32;  // S^T k-steps (32 d each)
  constexpr int NB = D / 16;   // PV output blocks (16 d each)
  using L = DecodeLds<D, KIND>;
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::kBytes];
  __shared__ float m_w[kDecodeWaves][16], l_w[kDecodeWaves][16];

  // ---- work item ----
  int w = blockIdx.x;
  const int split = w % max_splits;
  w /= max_splits;
  const int hc = w % n_hc;
  w /= n_hc;
  const int hk = w % Hkv;
  const int n = w / Hkv;
  const int G = Hq / Hkv;
  const int hq0 = hk * G + hc * 16;
  const int Gc = min(16, G - hc * 16);

  // a context longer than its block-table row is cut to the row (never read
  // past block_tables[n][max_blocks - 1])
  const int Lctx = (KIND == kKindContig16) ? S_contig
                                           : min(max(0, context_lens[n]), max_blocks * kDecodePage);
  const int n_pages = (Lctx + kDecodePage - 1) / kDecodePage;
  const int n_splits = max(1, (n_pages + kPagesPerSplit - 1) / kPagesPerSplit);
  if (split >= n_splits) return;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, grp = lane >> 4;
  const int p_begin = split * kPagesPerSplit + wave * kPagesPerWave;
  const int p_end = min(p_begin + kPagesPerWave, n_pages);
  const int n_steps = p_end > p_begin ? (p_end - p_begin + 1) / 2 : 0;

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

  // ---- page ids and per-page scales (lane j < 16 holds page p_begin + j) ----
  int pid_lane = 0;
  float ksc_lane = 1.f, vsc_lane = 1.f;
  if (KIND != kKindContig16) {
    if (l16 == lane && p_begin + lane < p_end) {
      pid_lane = block_tables[(size_t)n * max_blocks + p_begin + lane];
      pid_lane = min(max(pid_lane, 0), num_blocks - 1);
    }
    if (KIND == kKindPagedFp8) {
      if (per_block) {
        if (l16 == lane && p_begin + lane < p_end) {
          ksc_lane = k_scale[(size_t)pid_lane * Hkv + hk];
          vsc_lane = v_scale[(size_t)pid_lane * Hkv + hk];
        }
      } else {
        ksc_lane = k_scale[hk];
        vsc_lane = v_scale[hk];
      }
    }
  }

  unsigned char* wlds = lds + wave * L::kBytesPerWave;

  // ---- prefetch registers for one step (two pages) ----
  // K: paged 16-bit 4 x 16 B per page, paged fp8 2 x 16 B per page,
  //    contiguous: the K^T operand itself (NKS x 16 B per page)
  // V: paged: operand layout (16-bit: NB x 8 B, fp8: NB x 4 B per page),
  //    contiguous: 4 x 16 B per page of V rows (to LDS)
  // 16-byte chunks per lane for one page: 16-bit [D][16] = D/32, fp8 = D/64
  constexpr int KREG = KIND == kKindPaged16 ? D / 32 : KIND == kKindPagedFp8 ? D / 64 : NKS;
  u32x4 kreg[2][KREG];
  constexpr int VREG = KIND == kKindContig16 ? (16 * D * 2) / (64 * 16) : NB;
  u32x4 vreg_c[2][KIND == kKindContig16 ? VREG : 1];
  u32x2 vreg16[2][KIND == kKindPaged16 ? NB : 1];
  uint32_t vreg8[2][KIND == kKindPagedFp8 ? NB : 1];

  const size_t head_stride_pages = (size_t)D * 16;  // elements of one (page, head) chunk
  auto load_step = [&](int step) {
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
        for (int ks = 0; ks < NKS; ++ks) {
          if (valid && tok < S_contig)
            kreg[pp][ks] = *(const u32x4*)(Kp + (size_t)tok * D + 32 * ks + 8 * grp);
          else
            kreg[pp][ks] = u32x4{0, 0, 0, 0};
        }
        // V rows of the page: 16 rows x D, lanes take 16-byte chunks row-major
        constexpr int CH = D / 8;
#pragma unroll
        for (int i = 0; i < VREG; ++i) {
          const int c = lane + 64 * i;
          const int r = c / CH, col = (c % CH) * 8;
          const int vt = page * 16 + r;
          if (valid && vt < S_contig)
            vreg_c[pp][i] = *(const u32x4*)(Vp + (size_t)vt * D + col);
          else
            vreg_c[pp][i] = u32x4{0, 0, 0, 0};
        }
      } else {
        const int pid = __builtin_amdgcn_readlane(pid_lane, 2 * step + pp);
        const size_t chunk = ((size_t)pid * Hkv + hk) * head_stride_pages;
        if (KIND == kKindPaged16) {
          const uint16_t* Kp = (const uint16_t*)Kc + chunk;
          const uint16_t* Vp = (const uint16_t*)Vc + chunk;
#pragma unroll
          for (int i = 0; i < KREG; ++i)
            kreg[pp][i] = valid ? *(const u32x4*)(Kp + (lane + 64 * i) * 8) : u32x4{0, 0, 0, 0};
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            vreg16[pp][nb] = valid ? *(const u32x2*)(Vp + (16 * nb + l16) * 16 + 4 * grp) : u32x2{0, 0};
        } else {
          const unsigned char* Kp = (const unsigned char*)Kc + chunk;
          const unsigned char* Vp = (const unsigned char*)Vc + chunk;
#pragma unroll
          for (int i = 0; i < KREG; ++i)
            kreg[pp][i] = valid ? *(const u32x4*)(Kp + (lane + 64 * i) * 16) : u32x4{0, 0, 0, 0};
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            vreg8[pp][nb] = valid ? *(const uint32_t*)(Vp + (16 * nb + l16) * 16 + 4 * grp) : 0u;
        }
      }
    }
  };

  f32x4 o[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf, l_run = 0.f;

  if (n_steps > 0) load_step(0);
  for (int step = 0; step < n_steps; ++step) {
    // ---- stage this step's K (paged) or V (contiguous) into wave LDS ----
    if (KIND == kKindPaged16) {
      uint16_t* kl = (uint16_t*)wlds;
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
#pragma unroll
        for (int i = 0; i < KREG; ++i) {
          const int e = (lane + 64 * i) * 8;  // element offset in the [D][16] page
          const int row = e >> 4;
          *(u32x4*)(kl + pp * L::kPaged16PageElems + e + (row >> 3) * 64) = kreg[pp][i];
        }
    } else if (KIND == kKindPagedFp8) {
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
#pragma unroll
        for (int i = 0; i < KREG; ++i)
          *(u32x4*)(wlds + pp * D * 16 + (lane + 64 * i) * 16) = kreg[pp][i];
    } else {
      uint16_t* vl = (uint16_t*)wlds;
      constexpr int CH = D / 8;
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
#pragma unroll
        for (int i = 0; i < VREG; ++i) {
          const int c = lane + 64 * i;
          const int r = c / CH, col = (c % CH) * 8;
          *(u32x4*)(vl + (16 * pp + r) * (D + 16) + col) = vreg_c[pp][i];
        }
    }
    // keep this step's V operand / contiguous K operand before the prefetch
    // overwrites the registers
    u32x2 v16[2][KIND == kKindPaged16 ? NB : 1];
    uint32_t v8[2][KIND == kKindPagedFp8 ? NB : 1];
    u32x4 kc_cur[2][KIND == kKindContig16 ? NKS : 1];
    if (KIND == kKindPaged16) {
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) v16[pp][nb] = vreg16[pp][nb];
    } else if (KIND == kKindPagedFp8) {
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) v8[pp][nb] = vreg8[pp][nb];
    } else {
#pragma unroll
      for (int pp = 0; pp < 2; ++pp)
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) kc_cur[pp][ks] = kreg[pp][ks];
    }
    __builtin_amdgcn_wave_barrier();
    if (step + 1 < n_steps) load_step(step + 1);

    // ---- S^T per page ----
    f32x4 s[2];
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      s[pp] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        vec8 a;
        if (KIND == kKindPaged16) {
          // tr16: source lane (j = l16/4, c = l16%4) -> row 32ks + 8grp + 4r + j, col 4c
          const int row = 32 * ks + 8 * grp + (l16 >> 2);
          const uint16_t* kl = (const uint16_t*)wlds + pp * L::kPaged16PageElems;
          const uint16_t* p0 = kl + row * 16 + (row >> 3) * 64 + 4 * (l16 & 3);
          const int row4 = row + 4;
          const uint16_t* p1 = kl + row4 * 16 + (row4 >> 3) * 64 + 4 * (l16 & 3);
          const vec4 lo = Tr::tr_read((const CA_LDS void*)p0);
          const vec4 hi = Tr::tr_read((const CA_LDS void*)p1);
          a = cat4<vec8, vec4>(lo, hi);
        } else if (KIND == kKindPagedFp8) {
          // tr8: source lane (j = l16/2, c = l16%2) -> row 32ks + 8grp + j, col 8c
          const int row = 32 * ks + 8 * grp + (l16 >> 1);
          const i32x2 raw = tr8_read((const CA_LDS void*)(wlds + pp * D * 16 + row * 16 + 8 * (l16 & 1)));
          a = fp8x8_to<Tr>((uint32_t)raw[0], (uint32_t)raw[1]);
        } else {
          a = __builtin_bit_cast(vec8, kc_cur[pp][ks]);
        }
        s[pp] = Tr::mfma16(a, qv[ks], s[pp]);
      }
    }

    // ---- online softmax over the 32 tokens of the step ----
    const int pageA = p_begin + 2 * step;
    float cA = scale_log2, cB = scale_log2, vsA = 1.f, vsB = 1.f;
    if (KIND == kKindPagedFp8) {
      cA *= __shfl(ksc_lane, 2 * step, 64);
      cB *= __shfl(ksc_lane, 2 * step + 1, 64);
      vsA = __shfl(vsc_lane, 2 * step, 64);
      vsB = __shfl(vsc_lane, 2 * step + 1, 64);
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

    // ---- O += P V^T ----
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      vec8 bv;
      if (KIND == kKindPaged16) {
        const vec4 lo = __builtin_bit_cast(vec4, v16[0][nb]);
        const vec4 hi = __builtin_bit_cast(vec4, v16[1][nb]);
        bv = cat4<vec8, vec4>(lo, hi);
      } else if (KIND == kKindPagedFp8) {
        bv = fp8x8_to<Tr>(v8[0][nb], v8[1][nb]);
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
  }

  // ---- per-wave totals: l over the 4 lanes of a head; m is already uniform ----
  l_run = pair16_sum(l_run);
  l_run = pair32_sum(l_run);

  __syncthreads();  // staging LDS is reused for the merge
  float* om = (float*)lds;  // [wave][16][D]
  if (lane < 16) {
    m_w[wave][lane] = m_run;
    l_w[wave][lane] = l_run;
  }
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int r = 0; r < 4; ++r) om[(wave * 16 + 4 * grp + r) * D + 16 * nb + l16] = o[nb][r];
  __syncthreads();

  const bool single = (n_splits == 1);
  for (int idx = tid; idx < Gc * D; idx += kDecodeWaves * 64) {
    const int g = idx / D, d = idx % D;
    float M = kNegInf;
#pragma unroll
    for (int wv = 0; wv < kDecodeWaves; ++wv) M = __builtin_fmaxf(M, m_w[wv][g]);
    float lsum = 0.f, acc = 0.f;
    if (M != kNegInf) {
#pragma unroll
      for (int wv = 0; wv < kDecodeWaves; ++wv) {
        const float f = (m_w[wv][g] == kNegInf) ? 0.f : fast_exp2(m_w[wv][g] - M);
        lsum += l_w[wv][g] * f;
        acc += om[(wv * 16 + g) * D + d] * f;
      }
    }
    const float val = (lsum > 0.f) ? acc / lsum : 0.f;
    const int hq = hq0 + g;
    if (single) {
      const vec2 pk = Tr::pack2(val, 0.f);
      O[((size_t)n * Hq + hq) * D + d] = __builtin_bit_cast(uint16_t, pk[0]);
    } else {
      const size_t slot = ((size_t)n * Hq + hq) * max_splits + split;
      ws_o[slot * D + d] = val;
      if (d == 0) ws_lse[slot] = (lsum > 0.f) ? M + __log2f(lsum) : kNegInf;
    }
  }
}

// Combines the split partials of every (sequence, query head) with more than
// one split: o = sum_s 2^(lse_s - M) o_s / sum_s 2^(lse_s - M).
template <typename Tr, int D>
__global__ __launch_bounds__(D) void decode_merge_kernel(
    const int32_t* __restrict__ context_lens, int max_tokens, const float* __restrict__ ws_o,
    const float* __restrict__ ws_lse, uint16_t* __restrict__ O, int Hq, int max_splits) {
  using vec2 = typename Tr::vec2;
  const int n = blockIdx.x / Hq, hq = blockIdx.x % Hq;
  const int Lctx = context_lens ? min(max(0, context_lens[n]), max_tokens) : max_tokens;
  const int n_pages = (Lctx + kDecodePage - 1) / kDecodePage;
  const int n_splits = (n_pages + kPagesPerSplit - 1) / kPagesPerSplit;
  if (n_splits <= 1) return;
  const size_t slot0 = ((size_t)n * Hq + hq) * max_splits;
  const int d = threadIdx.x;
  float M = kNegInf;
  for (int s = 0; s < n_splits; ++s) M = __builtin_fmaxf(M, ws_lse[slot0 + s]);
  float wsum = 0.f, acc = 0.f;
  if (M != kNegInf) {
    for (int s = 0; s < n_splits; ++s) {
      const float lse = ws_lse[slot0 + s];
      const float f = (lse == kNegInf) ? 0.f : fast_exp2(lse - M);
      wsum += f;
      acc += f * ws_o[(slot0 + s) * D + d];
    }
  }
  const float val = wsum > 0.f ? acc / wsum : 0.f;
  const vec2 pk = Tr::pack2(val, 0.f);
  O[((size_t)n * Hq + hq) * D + d] = __builtin_bit_cast(uint16_t, pk[0]);
}

size_t decode_workspace_bytes(int N, int Hq, int D, int max_tokens) {
  const int pages = (max_tokens + kDecodePage - 1) / kDecodePage;
  const int max_splits = (pages + kPagesPerSplit - 1) / kPagesPerSplit;
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
  const int max_splits = max(1, (pages + kPagesPerSplit - 1) / kPagesPerSplit);
  const int G = Hq / Hkv;
  const int n_hc = (G + 15) / 16;
  const size_t need = decode_workspace_bytes(N, Hq, D, max_tokens);
  if (ws_bytes < need) return hipErrorInvalidValue;
  float* ws_o = (float*)ws;
  float* ws_lse = need ? ws_o + (size_t)N * Hq * max_splits * D : nullptr;
  const long long grid = (long long)N * Hkv * n_hc * max_splits;
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL((decode_split_kernel<Tr, D, KIND>), dim3((unsigned)grid),
                     dim3(kDecodeWaves * 64), 0, stream, (const uint16_t*)q, kc, vc, k_scale,
                     v_scale, per_block, bt, lens, (uint16_t*)out, ws_o, ws_lse, Hq, Hkv,
                     max_blocks, num_blocks, S_contig, max_splits, n_hc, scale * kLog2e);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || max_splits <= 1) return e;
  hipLaunchKernelGGL((decode_merge_kernel<Tr, D>), dim3((unsigned)(N * Hq)), dim3(D), 0, stream,
                     KIND == kKindContig16 ? nullptr : lens, max_tokens, ws_o, ws_lse,
                     (uint16_t*)out, Hq, max_splits);
  return hipGetLastError();
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
  return hipErrorInvalidValue;
}

}  // namespace ca
