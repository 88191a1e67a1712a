// Prefill (flash-attention forward) for gfx950: bf16/fp16 MFMA, K/V tiles in
// LDS, online softmax in registers.
//
// Computes O = softmax(Q K^T * scale [+ causal mask]) V per (batch, q-head),
// the contract of dispatch_flash_attention_v2 / _v3_hopper / fused_gqa in the
// reference (kernels_api.h:29-33,52-56,78-83; math flash_attention_v2_kernel.cuh:
// 82-83 causal tile bound, 179-229 online softmax, 223 l == 0 -> 0).
//
// Work decomposition
//   one workgroup = 8 waves = 256 query rows of one (b, h);
//   each wave owns 32 query rows for the whole KV walk;
//   KV tiles of 64 keys travel HBM -> LDS by buffer loads into a ring of 4
//   tiles (one barrier per tile) shared by the 8 waves.
// Per wave and KV tile (32x32x16 MFMAs):
//   S^T[64 keys x 32 q] = K Q^T   (A = K rows from LDS, B = Q from registers)
//   softmax over keys: keys live in the registers of a lane (16 per 32-key
//   block) and in its partner lane (lane ^ 32), so the row max is a register
//   max plus one cross-half exchange;
//   O^T[D x 32 q] += V^T P^T      (A = V^T via ds_read_b64_tr_b16 from the
//   row-major V tile, B = P^T straight from the S^T accumulator registers).
// Holding S and O transposed keeps a query's statistics (max, sum, rescale
// factor) in the lane that owns that query's column of O^T.
//
// Key permutation: the S^T A-operand lane i reads K row rho(i) (bits 2 and 3
// of i swapped). With the 32x32 accumulator layout (row 8*(r/4) + 4*half +
// r%4 in register r) this makes register r of lane half h hold key
// 16*(r/8) + 8*h + r%8, i.e. eight consecutive keys per PV k-step, exactly the
// B-operand layout of the PV MFMA — no LDS round trip for P.
#include <type_traits>

#include "common.h"
#include "launch.h"
#include "lds_dma.h"

namespace ca {

// MFMA blocks run at raised wave priority (s_setprio), so a wave's MFMAs win
// issue over its partner wave's softmax VALU on the same SIMD (+1-2.5 %
// measured at head dim 128).
#ifndef CA_PF_STALE
#define CA_PF_STALE 1
#endif
#ifndef CA_PF_PRIO
#define CA_PF_PRIO 1
#endif

// Rotate-half RoPE of the Q operand of query row `pos` in registers (the
// rotation of rope.hip, fused_rope_flash_attention_kernel.cuh:60-70): qv[ks]
// holds dims 16 ks + 8 hl + e, so dim c < D/2 and its partner c + D/2 sit in
// k-steps ks and ks + D/32 of the same lane.
template <typename Tr, int D>
__device__ __forceinline__ void rope_q(typename Tr::vec8 (&qv)[D / 16], RopeQ rq, int pos, int hl) {
  using vec2 = typename Tr::vec2;
  constexpr int H = D / 2, HKS = D / 32;
  const float* cr = rq.cos + (size_t)pos * D;
  const float* sr = rq.sin + (size_t)pos * D;
#pragma unroll
  for (int ks = 0; ks < HKS; ++ks) {
    const int c = 16 * ks + 8 * hl;
    float ca[8], sa[8], cb[8], sb[8];
#pragma unroll
    for (int h4 = 0; h4 < 8; h4 += 4) {
      *(float4*)(ca + h4) = *(const float4*)(cr + c + h4);
      *(float4*)(sa + h4) = *(const float4*)(sr + c + h4);
      *(float4*)(cb + h4) = *(const float4*)(cr + c + H + h4);
      *(float4*)(sb + h4) = *(const float4*)(sr + c + H + h4);
    }
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const float a0 = (float)qv[ks][e], a1 = (float)qv[ks][e + 1];
      const float b0 = (float)qv[ks + HKS][e], b1 = (float)qv[ks + HKS][e + 1];
      const vec2 lo = Tr::pack2(a0 * ca[e] - b0 * sa[e], a1 * ca[e + 1] - b1 * sa[e + 1]);
      const vec2 hi = Tr::pack2(b0 * cb[e] + a0 * sb[e], b1 * cb[e + 1] + a1 * sb[e + 1]);
      qv[ks][e] = lo[0];
      qv[ks][e + 1] = lo[1];
      qv[ks + HKS][e] = hi[0];
      qv[ks + HKS][e + 1] = hi[1];
    }
  }
}

// ---------------------------------------------------------------------------
// Head dim 64 and 128 kernel.
//
// One workgroup = BM query rows of one (b, h) (BM = 256 or 384), split over
// its waves: NH = 1 gives BM/32 waves of 32 rows (two or three per SIMD),
// NH = 2 waves of 64 rows. A wave owns NH 32-query halves; a K fragment read
// from LDS feeds the S^T MFMAs of all of them and a V^T fragment their O^T
// MFMAs, so LDS read bytes per FLOP fall as 1/NH. With CA_PF_AG the O^T
// accumulators, the S^T accumulators and Q live in AGPRs.
//
// K/V tiles of 64 keys travel HBM -> LDS with buffer loads into a ring of
// kStages tiles (the loaders share every K and V tile; one barrier per
// tile). Tile layout: 64 rows x 2D bytes, unpadded; the 16-byte chunk c of
// row r is stored at position c ^ swz(r), which makes both read patterns
// bank-conflict free:
//   K, ds_read_b128: a 16-lane group reads one chunk of 16 consecutive rows
//     -> 16 distinct bank positions;
//   V, ds_read_b64_tr_b16: a 32-lane group reads chunks 4ob..4ob+3 of 4
//     consecutive rows 4u..4u+3 -> 16 distinct bank positions.
// D = 128 (256-byte rows): swz(r) = 4*(r%4) + (r/4)%4, the position quad
// ob ^ (r%4) differs per row. D = 64 (128-byte rows, two per 256 bytes of
// banks): swz(r) = 4*((r/2)%2) + (r/4)%4 gives the 8 rows of one parity
// among 16 consecutive rows 8 distinct chunks, and rows r, r+2 opposite
// 4-chunk halves. D = 64 builds only the default schedule (NH = 1, no
// software pipeline).
// ---------------------------------------------------------------------------
template <int D>
struct PfGeom {
  static_assert(D == 64 || D == 128, "head dim");
  static constexpr int kBN = 64;                     // keys per tile
  static constexpr int kRowB = D * 2;                // bytes per K/V row
  static constexpr int kLpr = kRowB / 16;            // 16-byte chunks per row
  static constexpr int kRpk = 1024 / kRowB;          // rows per 1-KB load
  static constexpr int kTileB = kBN * kRowB;         // bytes per K (or V) tile
  static constexpr int kStageB = 2 * kTileB;         // K tile then V tile
  static constexpr int kNKS = D / 16;                // QK k-steps
  static constexpr int kNOB = D / 32;                // O^T row blocks
  __device__ static __forceinline__ int swz(int r) {
    return D == 128 ? (((r & 3) << 2) | ((r >> 2) & 3)) : ((((r >> 1) & 1) << 2) | ((r >> 2) & 3));
  }
};

// acc *= alpha on an accumulator kept in AGPRs, element by element through one
// VGPR, so the accumulator never needs a VGPR copy (a plain C++ multiply
// makes the compiler keep a VGPR image of every accumulator of the loop).
// The compiler does not see these AGPR accesses as dependent on the MFMAs
// that write the accumulators, so the caller brackets them with acc_gap().
__device__ __forceinline__ void scale_acc(f32x16& acc, float alpha) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float x = acc[r];
    float tmp;
    CA_DEVICE_ASM(
        "v_accvgpr_read_b32 %1, %0\n\t"
        "v_mul_f32 %1, %1, %2\n\t"
        "v_accvgpr_write_b32 %0, %1"
        : "+a"(x), "=&v"(tmp)
        : "v"(alpha));
    acc[r] = x;
  }
}
// 24 wait states: longer than any MFMA-result -> VALU and VALU -> MFMA-operand
// hazard of gfx950, so MFMAs issued before it have written their results.
__device__ __forceinline__ void acc_gap() { CA_DEVICE_ASM("s_nop 7\n\ts_nop 7\n\ts_nop 7"); }

// Per tile two phases, each pairing MFMAs with VALU work they do not depend
// on (order fixed with scheduling barriers):
//   PIPE (software pipeline across tiles):
//     A(t): S^T(t+1) = K(t+1) Q^T   with  P(t) = exp2(...) of the tile-t
//           logits held in VGPRs;
//     B(t): O^T += V(t)^T P(t)^T    with  copying S^T(t+1) out of the
//           accumulators, masking it and taking its row max;
//     after B(t) the running max and the (rare) O rescale for tile t+1 are
//     settled, so A(t+1) can exponentiate;
//   !PIPE: QK(t), max, exp, PV(t) in sequence; the overlap of MFMA and VALU
//     comes from the other wave on the SIMD (NH = 1).
// Waves per workgroup for BM query rows at 32*NH rows per wave, and the
// workgroups per CU that keep 2/NH waves on each SIMD.
constexpr int pf_waves(int bm, int nh) { return bm / (32 * nh); }
constexpr int pf_wg_per_cu(int bm, int nh) {
  return (8 / nh) / pf_waves(bm, nh) > 0 ? (8 / nh) / pf_waves(bm, nh) : 1;
}
#ifndef CA_PF_AG
#define CA_PF_AG 0
#endif
#ifndef CA_PF_PVX
#define CA_PF_PVX 0
#endif
#ifndef CA_PF_KDEPTH
#define CA_PF_KDEPTH 1
#endif
#ifndef CA_PF_VDEPTH
#define CA_PF_VDEPTH 2
#endif

// One query tile (kBM rows of head bh) of the workgroup: the whole key walk
// and the output store. On return every wave has waited for its own HBM ->
// LDS loads, but other waves may still read the ring.
template <typename Tr, int D, bool CAUSAL, bool POS, int NH, bool PIPE, int BM, int STAGES>
__device__ CA_INLINE void prefill_dma_qtile(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, uint16_t* __restrict__ O, float* __restrict__ Lse, int S, int Hq,
    int Hkv, float scale_log2, int bh, int qt, int q_shift, RopeQ rq) {
  using Gm = PfGeom<D>;
  using vec8 = typename Tr::vec8;
  using vec4 = typename Tr::vec4;
  using vec2 = typename Tr::vec2;
  constexpr int kBN = Gm::kBN, kRowB = Gm::kRowB, kTileB = Gm::kTileB, kStageB = Gm::kStageB;
  constexpr int kNKS = Gm::kNKS, kNOB = Gm::kNOB;
  static_assert(D == 128 || (NH == 1 && !PIPE && !CA_PF_AG), "D = 64: default schedule only");
  constexpr int kBM = BM;                        // query rows per workgroup
  constexpr int kStages = STAGES;                // K/V tiles in the LDS ring
  constexpr int kRW = 32 * NH;                   // query rows per wave
  constexpr int kNW = kBM / kRW;                 // waves per workgroup
  // waves that issue the HBM -> LDS loads: all of them when they divide the
  // 16 1-KB loads of a tile evenly, else the first 8
  // row max only on a wave's first tile (stale_softmax); 8-wave tiles (at
  // three waves per SIMD its rare path leaves too few registers)
  constexpr bool STALE = CA_PF_STALE != 0 && !PIPE && kNW == 8;
  constexpr int kLoaders = (kTileB / 1024) % kNW == 0 ? kNW : 8;
  constexpr int kDmaPerWave = kTileB / 1024 / kLoaders;  // 1 KB loads per loader per tile (K, and V)

  __shared__ __attribute__((aligned(1024))) unsigned char lds[kStages * kStageB];

  const int b = bh / Hq, h = bh % Hq;
  const int hk = h / (Hq / Hkv);
  const int q0 = qt * kBM - q_shift;  // tile 0 may start before row 0 (rows < 0 are padding)
  const uint16_t* Qp = Q + (size_t)(b * Hq + h) * S * D;
  uint16_t* Op = O + (size_t)(b * Hq + h) * S * D;
  const uint16_t* Kp = K + (size_t)(b * Hkv + hk) * S * D;
  const uint16_t* Vp = V + (size_t)(b * Hkv + hk) * S * D;

  const int lane = __builtin_amdgcn_workitem_id_x() & 63;
  const int wave = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_workitem_id_x() >> 6);
  const int l32 = lane & 31, hl = lane >> 5;
  const int qw0 = q0 + wave * kRW;
  int myq[NH];
#pragma unroll
  for (int nb = 0; nb < NH; ++nb) myq[nb] = qw0 + 32 * nb + l32;

  // Q as the B operand of S^T = K Q^T, one set per 32-query half.
  vec8 qv[NH][kNKS];
#pragma unroll
  for (int nb = 0; nb < NH; ++nb) {
#pragma unroll
    for (int ks = 0; ks < kNKS; ++ks) {
      if (myq[nb] >= 0 && myq[nb] < S) {
        qv[nb][ks] = *(const vec8*)(Qp + (size_t)myq[nb] * D + 16 * ks + 8 * hl);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[nb][ks][e] = 0;
      }
#if CA_PF_AG
      CA_DEVICE_ASM("" : "+a"(qv[nb][ks]));  // Q lives in AGPRs (an MFMA operand may)
#endif
    }
    if (rq.cos && myq[nb] >= 0 && myq[nb] < S) rope_q<Tr, D>(qv[nb], rq, myq[nb], hl);
  }

  const int kv_end = CAUSAL ? min(S, q0 + kBM) : S;
  const int n_tiles = (kv_end + kBN - 1) / kBN;
  // tiles this wave computes on (it still loads and synchronises for all)
  const int w_end = CAUSAL ? min(kv_end, qw0 + kRW) : kv_end;
  const int w_tiles = (qw0 + kRW > 0 && qw0 < S) ? (w_end + kBN - 1) / kBN : 0;

  // HBM -> LDS with buffer loads over the keys this workgroup needs
  // ([0, kv_end) of the (b, kv head) slice; rows past it read as zero, so
  // partial and trailing tiles need no clamp). Load i of this wave covers
  // tile rows kRpk*(kDmaPerWave*wave + i) + lane/kLpr; the lane fetches the
  // chunk that belongs at position lane % kLpr. Tile tt reads through
  // resources that start at its first row.
  const uint32_t kv_bytes = (uint32_t)kv_end * kRowB;
  uint32_t dma_off[kDmaPerWave];
#pragma unroll
  for (int i = 0; i < kDmaPerWave; ++i) {
    const int row = Gm::kRpk * (kDmaPerWave * wave + i) + lane / Gm::kLpr;
    dma_off[i] = row * kRowB + 16 * ((lane % Gm::kLpr) ^ Gm::swz(row));
  }
  const bool loader = kLoaders == kNW || wave < kLoaders;
  auto issue = [&](int tt) CA_INLINE {
    if (!loader) return;
    unsigned char* kdst = lds + (tt % kStages) * kStageB + wave * (kDmaPerWave * 1024);
    const uint32_t toff = (uint32_t)tt * kTileB;
    const __amdgpu_buffer_rsrc_t k_rsrc = make_rsrc_at(Kp, toff, kv_bytes);
    const __amdgpu_buffer_rsrc_t v_rsrc = make_rsrc_at(Vp, toff, kv_bytes);
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i) {
      dma16_buf(k_rsrc, (CA_LDS void*)(kdst + 1024 * i), dma_off[i]);
      dma16_buf(v_rsrc, (CA_LDS void*)(kdst + kTileB + 1024 * i), dma_off[i]);
    }
  };

  // LDS read addresses (bytes from the stage base).
  // K: lane reads row krow (+32 per key block), logical chunk 2*ks + hl.
  const int krow = (l32 & 0x13) | ((l32 & 4) << 1) | ((l32 & 8) >> 1);
  const int fk = Gm::swz(krow);
  const uint32_t kofs = krow * kRowB + 32 * (fk >> 1) + 16 * (hl ^ (fk & 1));  // ^ 32*ks
  // V^T: tr16 source lane -> row tr_row (+4 for the second read), logical
  // chunk 4*ob + c0, byte 8*(s16 & 1) of it.
  const int g16 = lane >> 4, s16 = lane & 15;
  const int tr_row = 8 * (g16 >> 1) + (s16 >> 2);
  const int c0 = 2 * (g16 & 1) + ((s16 & 3) >> 1);
  // D = 128: swz(tr_row + 4) == swz(tr_row) + 1 (tr_row % 8 < 4)
  const int fv = Gm::swz(tr_row);
  const int fv2 = D == 128 ? fv + 1 : Gm::swz(tr_row + 4);
  const uint32_t vofs1 = kTileB + tr_row * kRowB + 64 * (fv >> 2) + 16 * (c0 ^ (fv & 3)) + 8 * (s16 & 1);
  const uint32_t vofs2 =
      kTileB + (tr_row + 4) * kRowB + 64 * (fv2 >> 2) + 16 * (c0 ^ (fv2 & 3)) + 8 * (s16 & 1);
  const uint32_t lds0 = lds_off(lds);
  auto stage = [&](int tt) CA_INLINE { return lds0 + (uint32_t)((tt % kStages) * kStageB); };

  f32x16 o[kNOB][NH];  // O^T accumulators (AGPRs)
  f32x16 sacc[2][NH];  // S^T accumulators [mb][nb] of the tile being multiplied (AGPRs)
  float sv[NH][32];    // VGPR copy of the S^T being normalised: sv[nb][16mb + r]
  vec8 pb[NH][4];      // P^T, B operand of the O^T MFMAs
#pragma unroll
  for (int i = 0; i < kNOB; ++i)
#pragma unroll
    for (int nb = 0; nb < NH; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[i][nb][r] = 0.f;
  float m_run[NH], l_run[NH], msub[NH];
#pragma unroll
  for (int nb = 0; nb < NH; ++nb) { m_run[nb] = kNegInf; l_run[nb] = 0.f; msub[nb] = 0.f; }
  constexpr float kMaskVal = POS ? kNegInf : -kNegInf;  // raw logit whose scaled image is -inf

  // P for logit pair p (16 pairs per half: nb = p/16, P^T k-step kk = (p%16)/4,
  // logits 8kk + 2j, +1 with j = p%4; sv[nb][8kk + e] <-> P^T k-step kk)
  float psum[NH][2];
  auto exp_pair = [&](int p) CA_INLINE {
    const int nb = p >> 4, kk = (p >> 2) & 3, j = p & 3;
    const int i0 = 8 * kk + 2 * j;
    const float p0 = fast_exp2(__builtin_fmaf(sv[nb][i0], scale_log2, -msub[nb]));
    const float p1 = fast_exp2(__builtin_fmaf(sv[nb][i0 + 1], scale_log2, -msub[nb]));
    const vec2 pk = Tr::pack2(p0, p1);
    pb[nb][kk][2 * j] = pk[0];
    pb[nb][kk][2 * j + 1] = pk[1];
    psum[nb][j & 1] += p0 + p1;
  };
  // copy logit pair p (nb = p/16, logits i0 = 2*(p%16), +1) out of the
  // accumulators into sv (masked if MASK; a masked logit becomes the value
  // whose exponential is 0) and fold it into the row max
  float tm[NH][2];  // two partial row maxima (independent dependency chains)
  auto copy_pair = [&](int p, int k0, auto mask_tag) CA_INLINE {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int nb = p >> 4, i0 = 2 * (p & 15);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int i = i0 + e;
      float x = sacc[i >> 4][nb][i & 15];
      if (MASK) {
        const int key = k0 + 32 * (i >> 4) + 16 * ((i >> 3) & 1) + 8 * hl + (i & 7);
        if (key >= S || (CAUSAL && key > myq[nb])) x = kMaskVal;
      }
      if (PIPE) CA_DEVICE_ASM("" : "+v"(x));  // a real VGPR copy: the accumulators are reused
      sv[nb][i] = x;
    }
  };
  auto fold_max = [&](int p) CA_INLINE {
    const int nb = p >> 4, i0 = 2 * (p & 15);
    float& m = tm[nb][(p >> 1) & 1];
    m = POS ? __builtin_fmaxf(__builtin_fmaxf(m, sv[nb][i0]), sv[nb][i0 + 1])   // one v_max3
            : __builtin_fminf(__builtin_fminf(m, sv[nb][i0]), sv[nb][i0 + 1]);
  };
  auto take_pair = [&](int p, int k0, auto mask_tag) CA_INLINE {
    copy_pair(p, k0, mask_tag);
    fold_max(p);
  };
  // running max, lazy O rescale, exponent offset for the tile now in sv
  auto settle_max = [&]() CA_INLINE {
    float tmax[NH];
    bool any_need = false;
#pragma unroll
    for (int nb = 0; nb < NH; ++nb) {
      const float t2 = POS ? __builtin_fmaxf(tm[nb][0], tm[nb][1]) : __builtin_fminf(tm[nb][0], tm[nb][1]);
      tmax[nb] = pair32_max(t2 * scale_log2);
      any_need |= tmax[nb] > m_run[nb] + 8.0f;
    }
    if (__builtin_expect(wave_any(any_need), 0)) {  // rare: the max rose by > 2^8
      acc_gap();
#pragma unroll
      for (int nb = 0; nb < NH; ++nb) {
        const float m_new = __builtin_fmaxf(m_run[nb], tmax[nb]);
        const float alpha = (m_new == kNegInf) ? 1.f : fast_exp2(m_run[nb] - m_new);
#pragma unroll
        for (int i = 0; i < kNOB; ++i) {
#if CA_PF_AG
          scale_acc(o[i][nb], alpha);
#else
          o[i][nb] *= alpha;
#endif
        }
        l_run[nb] *= alpha;
        m_run[nb] = m_new;
      }
      acc_gap();
    }
#pragma unroll
    for (int nb = 0; nb < NH; ++nb) msub[nb] = (m_run[nb] == kNegInf) ? 0.f : m_run[nb];
  };

  // Softmax step of a tile after the wave's first, without its row max: the
  // exponentials are taken against the running max as it stands. They may
  // exceed 1 by far without harm as long as P stays representable in the
  // operand type of the PV MFMA (bf16: up to 2^48, with O and l far below
  // the float range; fp16: up to 2^15, its largest power of two below
  // 65504), so the max only has to be recomputed, O and l rescaled and the
  // exponentials taken again when some lane's tile sum passes that bound (or
  // is not finite). Saves the max3 tree and lane swap of every other tile.
  constexpr float kStaleMax = std::is_same<Tr, BF16>::value ? 0x1p48f : 0x1p15f;
  auto exp_all = [&]() CA_INLINE {
#pragma unroll
    for (int nb = 0; nb < NH; ++nb) psum[nb][0] = psum[nb][1] = 0.f;
#pragma unroll
    for (int p = 0; p < 16 * NH; ++p) exp_pair(p);
  };
  auto stale_softmax = [&](int tn, auto mask_tag) CA_INLINE {
#pragma unroll
    for (int p = 0; p < 16 * NH; ++p) copy_pair(p, tn * kBN, mask_tag);
    exp_all();
    bool big = false;
#pragma unroll
    for (int nb = 0; nb < NH; ++nb) big |= !(psum[nb][0] + psum[nb][1] <= kStaleMax);
    if (__builtin_expect(wave_any(big), 0)) {
#pragma unroll
      for (int nb = 0; nb < NH; ++nb) tm[nb][0] = tm[nb][1] = kMaskVal;
#pragma unroll
      for (int p = 0; p < 16 * NH; ++p) fold_max(p);
      settle_max();
      exp_all();
    }
#pragma unroll
    for (int nb = 0; nb < NH; ++nb) l_run[nb] += psum[nb][0] + psum[nb][1];
  };

  // Phase A: S^T(tn) = K(tn) Q^T (if QK), with the exponentials of the tile
  // in sv (if EXP) after the MFMAs, one pair each.
  auto phase_a = [&](int tn, auto qk_tag, auto exp_tag) CA_INLINE {
    constexpr bool QK = decltype(qk_tag)::value;
    constexpr bool EXP = decltype(exp_tag)::value;
#pragma unroll
    for (int nb = 0; nb < NH; ++nb) psum[nb][0] = psum[nb][1] = 0.f;
    if (QK) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < NH; ++nb)
#pragma unroll
          for (int r = 0; r < 16; ++r) sacc[mb][nb][r] = 0.f;
      if (CA_PF_PRIO) __builtin_amdgcn_s_setprio(1);
      const uint32_t ka = stage(tn) + kofs;
      // K fragments of KD k-steps in flight ahead of the MFMAs (ring of KD + 1)
      constexpr int KD = CA_PF_KDEPTH;
      u32x4 kr[KD + 1][2];
      auto kread = [&](int ks) CA_INLINE {
        const uint32_t an = ka ^ (32 * ks);
        kr[ks % (KD + 1)][0] = lds_read_b128<0>(an);
        kr[ks % (KD + 1)][1] = lds_read_b128<32 * kRowB>(an);
      };
#pragma unroll
      for (int ks = 0; ks < KD; ++ks) kread(ks);
#pragma unroll
      for (int ks = 0; ks < kNKS; ++ks) {
        const int cb = ks % (KD + 1);
        if (ks + KD < kNKS) kread(ks + KD);
        wait_lgkm_n(2 * (KD < kNKS - 1 - ks ? KD : kNKS - 1 - ks));  // k-step ks landed
        after_wait(kr[cb][0]);
        after_wait(kr[cb][1]);
#pragma unroll
        for (int j = 0; j < 2 * NH; ++j) {
          const int mb = j / NH, nb = j % NH;
          const vec8 a = __builtin_bit_cast(vec8, kr[cb][mb]);
          sacc[mb][nb] = Tr::mfma32(a, qv[nb][ks], sacc[mb][nb]);
          if (EXP) exp_pair(2 * NH * ks + j);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);  // then the pair's VALU
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (CA_PF_PRIO) __builtin_amdgcn_s_setprio(0);
    } else if (EXP) {
#pragma unroll
      for (int p = 0; p < 16 * NH; ++p) exp_pair(p);
    }
    if (EXP) {
#pragma unroll
      for (int nb = 0; nb < NH; ++nb) l_run[nb] += psum[nb][0] + psum[nb][1];
    }
  };

  // Phase B: O^T += V(t)^T P^T (if PV), with S^T(tn) taken out of the
  // accumulators (if NEXT; masked if MASK) after the MFMAs; then settle.
  auto phase_b = [&](int t, int tn, auto pv_tag, auto next_tag, auto mask_tag) CA_INLINE {
    constexpr bool PV = decltype(pv_tag)::value;
    constexpr bool NEXT = decltype(next_tag)::value;
    const int k0n = tn * kBN;
#pragma unroll
    for (int nb = 0; nb < NH; ++nb) tm[nb][0] = tm[nb][1] = kMaskVal;
    if (PV) {
      if (CA_PF_PRIO) __builtin_amdgcn_s_setprio(1);
      const uint32_t va1 = stage(t) + vofs1, va2 = stage(t) + vofs2;
      // V^T fragments of VD k-steps in flight ahead of the MFMAs (ring of VD + 1)
      constexpr int VD = CA_PF_VDEPTH;
      u32x2 vr[VD + 1][2];
      // step st: O^T block ob, P^T k-step kk; with PVX consecutive MFMAs go
      // to different accumulators (a lone wave then issues them back to back)
      constexpr int NST = 4 * kNOB;  // steps: kNOB O^T blocks x 4 P^T k-steps
      auto st_ob = [](int st) CA_INLINE { return CA_PF_PVX ? (st % kNOB) : (st >> 2); };
      auto st_kk = [](int st) CA_INLINE { return CA_PF_PVX ? (st / kNOB) : (st & 3); };
      constexpr int kKK = 16 * kRowB;  // bytes per P^T k-step of V rows
      auto vread = [&](int st, int buf) CA_INLINE {
        const uint32_t x = 64 * st_ob(st);
        switch (st_kk(st)) {
          case 0: vr[buf][0] = lds_read_tr16<0>(va1 ^ x); vr[buf][1] = lds_read_tr16<0>(va2 ^ x); break;
          case 1: vr[buf][0] = lds_read_tr16<kKK>(va1 ^ x); vr[buf][1] = lds_read_tr16<kKK>(va2 ^ x); break;
          case 2: vr[buf][0] = lds_read_tr16<2 * kKK>(va1 ^ x); vr[buf][1] = lds_read_tr16<2 * kKK>(va2 ^ x); break;
          default: vr[buf][0] = lds_read_tr16<3 * kKK>(va1 ^ x); vr[buf][1] = lds_read_tr16<3 * kKK>(va2 ^ x); break;
        }
      };
#pragma unroll
      for (int st = 0; st < VD; ++st) vread(st, st);
#pragma unroll
      for (int st = 0; st < NST; ++st) {
        const int cb = st % (VD + 1);
        if (st + VD < NST) vread(st + VD, (st + VD) % (VD + 1));
        wait_lgkm_n(2 * (VD < NST - 1 - st ? VD : NST - 1 - st));  // step st landed
        after_wait(vr[cb][0]);
        after_wait(vr[cb][1]);
        const int ob = st_ob(st), kk = st_kk(st);
        u32x4 w4 = {vr[cb][0][0], vr[cb][0][1], vr[cb][1][0], vr[cb][1][1]};
        const vec8 a = __builtin_bit_cast(vec8, w4);
#pragma unroll
        for (int nb = 0; nb < NH; ++nb) {
          o[ob][nb] = Tr::mfma32(a, pb[nb][kk], o[ob][nb]);
          if (NEXT) take_pair(NH * st + nb, k0n, mask_tag);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (CA_PF_PRIO) __builtin_amdgcn_s_setprio(0);
    } else if (NEXT) {
#pragma unroll
      for (int p = 0; p < 16 * NH; ++p) take_pair(p, k0n, mask_tag);
    }
    if (NEXT) settle_max();
  };

  // ---- the tile walk ----------------------------------------------------------
  // Every wave walks all n_tiles tiles (it loads its share of each and meets
  // the others at the per-tile barrier). Only a wave's last tile can need a
  // mask (bounds or causal diagonal); it is masked when taken out of the
  // accumulators.
  using T_ = std::true_type;
  using F_ = std::false_type;
  constexpr int DIST = kStages - 1;  // tiles in flight ahead of the one waited for
#pragma unroll
  for (int tt = 0; tt < DIST; ++tt) issue(tt);
  // Barrier t: every wave has its loads of tile t + LEAD resident (PIPE: A(t)
  // reads K(t+1)) and is past its last read of tile t - 1, whose slot then
  // takes tile t + DIST.
  constexpr int LEAD = PIPE ? 1 : 0;
  auto sync = [&](int t) CA_INLINE {
    if (loader) wait_vmcnt<2 * kDmaPerWave * (DIST - 1 - LEAD)>();  // this wave's loads landed
    __builtin_amdgcn_s_barrier();                      // ... and every wave's
    issue(t + DIST);
  };
  int t = 0;
  if (PIPE) {
    if (loader) wait_vmcnt<2 * kDmaPerWave * (kStages - 2)>();  // tile 0 landed (this wave's part)
    __builtin_amdgcn_s_barrier();                   // ... and every wave's
    if (w_tiles > 0) {
      phase_a(0, T_{}, F_{});             // S^T(0)
      phase_b(-1, 0, F_{}, T_{}, T_{});   // its max (mask test exact for any tile)
    }
    for (; t + 2 < w_tiles; ++t) {  // next tile is not the wave's last
      sync(t);
      phase_a(t + 1, T_{}, T_{});
      phase_b(t, t + 1, T_{}, T_{}, F_{});
    }
    if (t + 2 == w_tiles) {  // next tile is the wave's last: mask it
      sync(t);
      phase_a(t + 1, T_{}, T_{});
      phase_b(t, t + 1, T_{}, T_{}, T_{});
      ++t;
    }
    if (t + 1 == w_tiles) {  // the wave's last tile
      sync(t);
      phase_a(-1, F_{}, T_{});
      phase_b(t, -1, T_{}, F_{}, F_{});
      ++t;
    }
  } else if (STALE) {
    // the wave's first tile takes the full max; later tiles stale_softmax
    if (w_tiles > 1) {
      sync(0);
      phase_a(0, T_{}, F_{});
      phase_b(-1, 0, F_{}, T_{}, F_{});
      phase_a(-1, F_{}, T_{});
      phase_b(0, -1, T_{}, F_{}, F_{});
      t = 1;
    }
    for (; t + 1 < w_tiles; ++t) {
      sync(t);
      phase_a(t, T_{}, F_{});
      stale_softmax(t, F_{});
      phase_b(t, -1, T_{}, F_{}, F_{});
    }
    if (t + 1 == w_tiles) {  // the wave's last tile, masked
      sync(t);
      phase_a(t, T_{}, F_{});
      if (t == 0) {
        phase_b(-1, t, F_{}, T_{}, T_{});
        phase_a(-1, F_{}, T_{});
      } else {
        stale_softmax(t, T_{});
      }
      phase_b(t, -1, T_{}, F_{}, F_{});
      ++t;
    }
  } else {
    for (; t + 1 < w_tiles; ++t) {
      sync(t);
      phase_a(t, T_{}, F_{});
      phase_b(-1, t, F_{}, T_{}, F_{});
      phase_a(-1, F_{}, T_{});
      phase_b(t, -1, T_{}, F_{}, F_{});
    }
    if (t + 1 == w_tiles) {  // the wave's last tile, masked
      sync(t);
      phase_a(t, T_{}, F_{});
      phase_b(-1, t, F_{}, T_{}, T_{});
      phase_a(-1, F_{}, T_{});
      phase_b(t, -1, T_{}, F_{}, F_{});
      ++t;
    }
  }
  for (; t < n_tiles; ++t) sync(t);
  wait_vmcnt<0>();  // no load may still target this workgroup's LDS when it exits
  acc_gap();

#pragma unroll
  for (int nb = 0; nb < NH; ++nb) {
    const float l_tot = pair32_sum(l_run[nb]);
    const float inv = (l_tot > 0.f) ? 1.f / l_tot : 0.f;
    if (Lse && hl == 0 && myq[nb] >= 0 && myq[nb] < S)
      Lse[(size_t)(b * Hq + h) * S + myq[nb]] = row_lse(m_run[nb], l_tot);
    if (myq[nb] >= 0 && myq[nb] < S) {
#pragma unroll
      for (int ob = 0; ob < kNOB; ++ob) {
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const int d = 32 * ob + 8 * a + 4 * hl;
          const vec2 lo = Tr::pack2(o[ob][nb][4 * a] * inv, o[ob][nb][4 * a + 1] * inv);
          const vec2 hi = Tr::pack2(o[ob][nb][4 * a + 2] * inv, o[ob][nb][4 * a + 3] * inv);
          vec4 w;
          w[0] = lo[0]; w[1] = lo[1]; w[2] = hi[0]; w[3] = hi[1];
          *(vec4*)(Op + (size_t)myq[nb] * D + d) = w;
        }
      }
    }
  }
}

template <typename Tr, int D, bool CAUSAL, bool POS, int NH, bool PIPE, int BM, int STAGES>
__global__ __launch_bounds__(64 * pf_waves(BM, NH), pf_wg_per_cu(BM, NH)) void prefill_dma_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, uint16_t* __restrict__ O, float* __restrict__ Lse, int S, int Hq,
    int Hkv, float scale_log2, int n_qt, int n_bh, int n_work, int paired, int q_shift, RopeQ rq) {
  const QTileWork wk =
      prefill_work(xcd_remap(__builtin_amdgcn_workgroup_id_x(), n_work), n_qt, n_bh, paired);
  const int n_pass = wk.qt1 < 0 ? 1 : 2;
#pragma clang loop unroll(disable)
  for (int pass = 0; pass < n_pass; ++pass) {
    // the second tile refills the LDS ring: every wave must be done reading it
    if (pass) __builtin_amdgcn_s_barrier();
    prefill_dma_qtile<Tr, D, CAUSAL, POS, NH, PIPE, BM, STAGES>(
        Q, K, V, O, Lse, S, Hq, Hkv, scale_log2, pass ? wk.bh1 : wk.bh0, pass ? wk.qt1 : wk.qt0, q_shift,
        rq);
  }
}

#ifndef CA_PF_NH
#define CA_PF_NH 1
#endif
#ifndef CA_PF_PIPE
#define CA_PF_PIPE 0
#endif
#ifndef CA_PF_MAXSTAGES
#define CA_PF_MAXSTAGES 4
#endif

template <typename Tr, int D, bool CAUSAL, int BM>
static hipError_t launch_prefill_dma_bm(const void* q, const void* k, const void* v, void* o, float* lse,
                                        int B, int Hq, int Hkv, int S, float scale,
                                        hipStream_t stream, RopeQ rq) {
  using Gm = PfGeom<D>;
  constexpr int NH = D == 128 ? CA_PF_NH : 1;
  constexpr bool PIPE = D == 128 && CA_PF_PIPE;
  // LDS ring: as many stages (32 KB at D = 128) as fit next to the other
  // workgroups on the CU
  constexpr int kLdsPerWg = 160 * 1024 / pf_wg_per_cu(BM, NH);
  constexpr int STAGES = kLdsPerWg / Gm::kStageB > CA_PF_MAXSTAGES ? CA_PF_MAXSTAGES
                                                                   : kLdsPerWg / Gm::kStageB;
  static_assert(STAGES >= (PIPE ? 3 : 2), "LDS ring too short for the schedule");
  const int n_qt = (S + BM - 1) / BM;
  // the padding rows of a ragged S go before row 0, in whole key tiles (so a
  // wave's causal diagonal still lies in one key tile): the partial tile is
  // the first one, whose causal key walk is the shortest
  const int q_shift = (n_qt * BM - S) / Gm::kBN * Gm::kBN;
  int paired = 0;
  const long long grid = prefill_grid(B, Hq, n_qt, CAUSAL, pf_wg_per_cu(BM, NH), &paired);
  if (grid == 0) return hipSuccess;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  const float sl2 = scale * kLog2e;
  const dim3 block(64 * pf_waves(BM, NH));
  if (sl2 >= 0.f) {
    hipLaunchKernelGGL((prefill_dma_kernel<Tr, D, CAUSAL, true, NH, PIPE, BM, STAGES>),
                       dim3((unsigned)grid), block, 0, stream, (const uint16_t*)q,
                       (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, lse, S, Hq, Hkv, sl2,
                       n_qt, B * Hq, (int)grid, paired, q_shift, rq);
  } else {
    hipLaunchKernelGGL((prefill_dma_kernel<Tr, D, CAUSAL, false, NH, PIPE, BM, STAGES>),
                       dim3((unsigned)grid), block, 0, stream, (const uint16_t*)q,
                       (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, lse, S, Hq, Hkv, sl2,
                       n_qt, B * Hq, (int)grid, paired, q_shift, rq);
  }
  return hipGetLastError();
}

// Workgroup height: 256 query rows (8 waves, two per SIMD). 384 rows (12
// waves, three per SIMD) measured +4-6 % at S = 3072 before the stale-max
// softmax, which only the 8-wave kernel can afford in registers and which
// gains more; the 384-row choice (when such tiles cover S with at most ~5 %
// padding and the grid gives every CU two workgroups) remains for builds
// without it.
template <typename Tr, int D, bool CAUSAL>
static hipError_t launch_prefill_dma(const void* q, const void* k, const void* v, void* o, float* lse,
                                     int B, int Hq, int Hkv, int S, float scale,
                                     hipStream_t stream, RopeQ rq) {
#ifdef CA_PF_BM
  return launch_prefill_dma_bm<Tr, D, CAUSAL, CA_PF_BM>(q, k, v, o, lse, B, Hq, Hkv, S, scale, stream, rq);
#else
  const long long n384 = (S + 383) / 384;
  const bool fits = n384 * 384 * 20 <= (long long)S * 21;
  const bool tall = !CA_PF_STALE && fits && (long long)B * Hq * n384 >= 2LL * device_cus();
  return tall ? launch_prefill_dma_bm<Tr, D, CAUSAL, 384>(q, k, v, o, lse, B, Hq, Hkv, S, scale, stream, rq)
              : launch_prefill_dma_bm<Tr, D, CAUSAL, 256>(q, k, v, o, lse, B, Hq, Hkv, S, scale, stream, rq);
#endif
}

hipError_t launch_prefill(int dtype, const void* q, const void* k, const void* v, void* o, float* lse,
                          int B, int Hq, int Hkv, int S, int D, float scale, bool causal,
                          hipStream_t stream, RopeQ rq) {
#define CA_PREFILL_DMA(TR, DD)                                                                    \
  if (D == DD) {                                                                                  \
    return causal ? launch_prefill_dma<TR, DD, true>(q, k, v, o, lse, B, Hq, Hkv, S, scale, stream, rq)  \
                  : launch_prefill_dma<TR, DD, false>(q, k, v, o, lse, B, Hq, Hkv, S, scale, stream, rq); \
  }
  if (dtype == kDtypeF32) return launch_prefill_f32(q, k, v, o, lse, B, Hq, Hkv, S, D, scale, causal, stream);
  if (dtype == kDtypeBF16) {
    CA_PREFILL_DMA(BF16, 64)
    CA_PREFILL_DMA(BF16, 128)
  } else if (dtype == kDtypeF16) {
    CA_PREFILL_DMA(F16, 64)
    CA_PREFILL_DMA(F16, 128)
  }
#undef CA_PREFILL_DMA
  return hipErrorInvalidValue;
}

}  // namespace ca
