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
//   tiles (one barrier per two tiles) shared by the 8 waves.
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
// One workgroup = 256 query rows of one (b, h) = 8 waves of 32 rows, two per
// SIMD (waves w and w+4 share one). K/V tiles of 64 keys travel HBM -> LDS
// with buffer loads into a ring of kStages tiles (every wave loads 1/8 of
// every K and V tile; one barrier per two tiles). Tile layout: 64 rows x 2D bytes,
// unpadded; the 16-byte chunk c of row r is stored at position c ^ swz(r),
// which makes both read patterns bank-conflict free:
//   K, ds_read_b128: a 16-lane group reads one chunk of 16 consecutive rows
//     -> 16 distinct bank positions;
//   V, ds_read_b64_tr_b16: a 32-lane group reads chunks 4ob..4ob+3 of 4
//     consecutive rows 4u..4u+3 -> 16 distinct bank positions.
// D = 128 (256-byte rows): swz(r) = 4*(r%4) + (r/4)%4, the position quad
// ob ^ (r%4) differs per row. D = 64 (128-byte rows, two per 256 bytes of
// banks): swz(r) = 4*((r/2)%2) + (r/4)%4 gives the 8 rows of one parity
// among 16 consecutive rows 8 distinct chunks, and rows r, r+2 opposite
// 4-chunk halves.
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

constexpr int kPfRows = 256;   // query rows per workgroup
constexpr int kPfWaves = 8;    // waves per workgroup (32 query rows each)
constexpr int kPfStages = 4;   // K/V tiles in the LDS ring (32 KB each at D = 128)
constexpr int kPfKDepth = 1;   // K fragments read ahead of the QK MFMAs (k-steps)
constexpr int kPfVDepth = 2;   // V^T fragments read ahead of the PV MFMAs (steps)
// Key tiles per workgroup barrier: one barrier every two tiles lets a
// SIMD's two waves drift apart within the pair instead of meeting after
// every PV (C2 +1.5 % over one barrier per tile, same box).
constexpr int kPfGroup = 2;
// 24 wait states: longer than any MFMA-result -> VALU and VALU -> MFMA-operand
// hazard of gfx950, so MFMAs issued before it have written their results.
__device__ __forceinline__ void acc_gap() { CA_DEVICE_ASM("s_nop 7\n\ts_nop 7\n\ts_nop 7"); }

// One query tile (256 rows of head bh) of the workgroup: the whole key walk
// and the output store. Per wave and KV tile: QK (16 MFMAs at D = 128), the
// softmax step, PV (16 MFMAs); the overlap of MFMA and VALU comes from the
// other wave on the SIMD. MFMA blocks run at raised wave priority
// (s_setprio), so a wave's MFMAs win issue over its partner wave's softmax
// VALU. On return every wave has waited for its own HBM -> LDS loads, but
// other waves may still read the ring.
template <typename Tr, int D, bool CAUSAL, bool POS>
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
  constexpr int kBM = kPfRows, kStages = kPfStages, kNW = kPfWaves;
  constexpr int kDmaPerWave = kTileB / 1024 / kNW;  // 1 KB loads per wave per tile (K, and V)
  static_assert(kDmaPerWave >= 1 && kTileB % (1024 * kNW) == 0, "tile loads");

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
  const int qw0 = q0 + wave * 32;
  const int myq = qw0 + l32;

  // Q as the B operand of S^T = K Q^T
  vec8 qv[kNKS];
#pragma unroll
  for (int ks = 0; ks < kNKS; ++ks) {
    if (myq >= 0 && myq < S) {
      qv[ks] = *(const vec8*)(Qp + (size_t)myq * D + 16 * ks + 8 * hl);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qv[ks][e] = 0;
    }
  }
  if (rq.cos && myq >= 0 && myq < S) rope_q<Tr, D>(qv, rq, myq, hl);

  const int kv_end = CAUSAL ? min(S, q0 + kBM) : S;
  const int n_tiles = (kv_end + kBN - 1) / kBN;
  // tiles this wave computes on (it still loads and synchronises for all)
  const int w_end = CAUSAL ? min(kv_end, qw0 + 32) : kv_end;
  const int w_tiles = (qw0 + 32 > 0 && qw0 < S) ? (w_end + kBN - 1) / kBN : 0;

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
  auto issue = [&](int tt) CA_INLINE {
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
  // load j of tile tt alone (j < kDmaPerWave: K, else V), in the same order
  // as issue()
  constexpr int kLoads = 2 * kDmaPerWave;
  auto issue_one = [&](int tt, int j) CA_INLINE {
    unsigned char* kdst = lds + (tt % kStages) * kStageB + wave * (kDmaPerWave * 1024);
    const uint32_t toff = (uint32_t)tt * kTileB;
    const int i = j >> 1;
    if ((j & 1) == 0)
      dma16_buf(make_rsrc_at(Kp, toff, kv_bytes), (CA_LDS void*)(kdst + 1024 * i), dma_off[i]);
    else
      dma16_buf(make_rsrc_at(Vp, toff, kv_bytes), (CA_LDS void*)(kdst + kTileB + 1024 * i), dma_off[i]);
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

  f32x16 o[kNOB];   // O^T accumulators
  f32x16 sacc[2];   // S^T accumulators [key block] of the tile being multiplied
  float sv[32];     // the S^T being normalised: sv[16 mb + r]
  vec8 pb[4];       // P^T, B operand of the O^T MFMAs
#pragma unroll
  for (int i = 0; i < kNOB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
  float m_run = kNegInf, l_run = 0.f, msub = 0.f;
  constexpr float kMaskVal = POS ? kNegInf : -kNegInf;  // raw logit whose scaled image is -inf

  // P for logit pair p (16 pairs: P^T k-step kk = p/4, logits 8kk + 2j, +1
  // with j = p%4; sv[8kk + e] <-> P^T k-step kk); two partial row sums
  float psum[2];
  auto exp_pair = [&](int p) CA_INLINE {
    const int kk = p >> 2, j = p & 3;
    const int i0 = 8 * kk + 2 * j;
    const float p0 = fast_exp2(__builtin_fmaf(sv[i0], scale_log2, -msub));
    const float p1 = fast_exp2(__builtin_fmaf(sv[i0 + 1], scale_log2, -msub));
    const vec2 pk = Tr::pack2(p0, p1);
    pb[kk][2 * j] = pk[0];
    pb[kk][2 * j + 1] = pk[1];
    psum[j & 1] += p0 + p1;
  };
  auto exp_all = [&]() CA_INLINE {
    psum[0] = psum[1] = 0.f;
#pragma unroll
    for (int p = 0; p < 16; ++p) exp_pair(p);
  };
  // copy logit pair p (logits 2p, 2p+1) out of the accumulators into sv
  // (masked if MASK: a masked logit becomes the value whose exponential is 0)
  auto copy_pair = [&](int p, int k0, auto mask_tag) CA_INLINE {
    constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int i = 2 * p + e;
      float x = sacc[i >> 4][i & 15];
      if (MASK) {
        const int key = k0 + 32 * (i >> 4) + 16 * ((i >> 3) & 1) + 8 * hl + (i & 7);
        if (key >= S || (CAUSAL && key > myq)) x = kMaskVal;
      }
      sv[i] = x;
    }
  };
  float tm[2];  // two partial row maxima (independent dependency chains)
  auto fold_max = [&](int p) CA_INLINE {
    float& m = tm[(p >> 1) & 1];
    m = POS ? __builtin_fmaxf(__builtin_fmaxf(m, sv[2 * p]), sv[2 * p + 1])   // one v_max3
            : __builtin_fminf(__builtin_fminf(m, sv[2 * p]), sv[2 * p + 1]);
  };
  // running max, lazy O rescale, exponent offset for the tile now in sv
  auto settle_max = [&]() CA_INLINE {
    const float t2 = POS ? __builtin_fmaxf(tm[0], tm[1]) : __builtin_fminf(tm[0], tm[1]);
    const float tmax = pair32_max(t2 * scale_log2);
    if (__builtin_expect(wave_any(tmax > m_run + 8.0f), 0)) {  // rare: the max rose by > 2^8
      acc_gap();
      const float m_new = __builtin_fmaxf(m_run, tmax);
      const float alpha = (m_new == kNegInf) ? 1.f : fast_exp2(m_run - m_new);
#pragma unroll
      for (int i = 0; i < kNOB; ++i) o[i] *= alpha;
      l_run *= alpha;
      m_run = m_new;
      acc_gap();
    }
    msub = (m_run == kNegInf) ? 0.f : m_run;
  };
  // Softmax step of the wave's first tile: the full row max first.
  auto first_softmax = [&](int tn, auto mask_tag) CA_INLINE {
    tm[0] = tm[1] = kMaskVal;
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      copy_pair(p, tn * kBN, mask_tag);
      fold_max(p);
    }
    settle_max();
    exp_all();
    l_run += psum[0] + psum[1];
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
  auto stale_softmax = [&](int tn, auto mask_tag) CA_INLINE {
#pragma unroll
    for (int p = 0; p < 16; ++p) copy_pair(p, tn * kBN, mask_tag);
    exp_all();
    if (__builtin_expect(wave_any(!(psum[0] + psum[1] <= kStaleMax)), 0)) {
      tm[0] = tm[1] = kMaskVal;
#pragma unroll
      for (int p = 0; p < 16; ++p) fold_max(p);
      settle_max();
      exp_all();
    }
    l_run += psum[0] + psum[1];
  };

  // S^T(tn) = K(tn) Q^T, K fragments kPfKDepth k-steps ahead of the MFMAs
  // The wave's loads of tile tn + kStages - kPfGroup (if past the first
  // kStages tiles, which are issued up front) go out between its k-steps,
  // one after every kNKS / kLoads of them: issued all at once after the
  // barrier, the 8 waves' loads queue behind each other (C2 +1.8 %).
  constexpr int kAhead = kStages - kPfGroup;
  auto qk = [&](int tn) CA_INLINE {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[mb][r] = 0.f;
    __builtin_amdgcn_s_setprio(1);
    const uint32_t ka = stage(tn) + kofs;
    constexpr int KD = kPfKDepth;
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
      for (int mb = 0; mb < 2; ++mb) {
        sacc[mb] = Tr::mfma32(__builtin_bit_cast(vec8, kr[cb][mb]), qv[ks], sacc[mb]);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);  // then up to 8 VALU
      }
      if (ks % (kNKS / kLoads) == kNKS / kLoads - 1 && tn + kAhead >= kStages)
        issue_one(tn + kAhead, ks / (kNKS / kLoads));
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // O^T += V(t)^T P^T, V^T fragments kPfVDepth steps ahead of the MFMAs
  auto pv = [&](int t) CA_INLINE {
    __builtin_amdgcn_s_setprio(1);
    const uint32_t va1 = stage(t) + vofs1, va2 = stage(t) + vofs2;
    constexpr int VD = kPfVDepth;
    u32x2 vr[VD + 1][2];
    constexpr int NST = 4 * kNOB;    // steps: kNOB O^T blocks x 4 P^T k-steps
    constexpr int kKK = 16 * kRowB;  // bytes per P^T k-step of V rows
    auto vread = [&](int st, int buf) CA_INLINE {
      const uint32_t x = 64 * (st >> 2);
      switch (st & 3) {
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
      const int ob = st >> 2, kk = st & 3;
      u32x4 w4 = {vr[cb][0][0], vr[cb][0][1], vr[cb][1][0], vr[cb][1][1]};
      o[ob] = Tr::mfma32(__builtin_bit_cast(vec8, w4), pb[kk], o[ob]);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // ---- the tile walk ----------------------------------------------------------
  // Every wave walks all n_tiles tiles (it loads its share of each and meets
  // the others at the barrier of every tile pair). Only a wave's last tile can need a
  // mask (bounds or causal diagonal); it is masked when taken out of the
  // accumulators. The wave's first tile takes the full row max, later tiles
  // the stale-max step.
  using T_ = std::true_type;
  using F_ = std::false_type;
#pragma unroll
  for (int tt = 0; tt < kStages; ++tt) issue(tt);
  // Barrier at tile t (t % kPfGroup == 0): every wave has its loads of tiles
  // t .. t + kPfGroup - 1 resident and is past its last read of tile t - 1,
  // so the slots of tiles t - kPfGroup .. t - 1 take tiles t + kAhead .. A
  // wave that computes on tile t issues tile t + kAhead's loads inside qk(t);
  // one that does not, in sync(t, true). Loads issued after the group's:
  // kStages - kPfGroup tiles at t = 0 (the up-front ones), kStages -
  // 2 kPfGroup after that.
  auto sync = [&](int t, bool load_here) CA_INLINE {
    if (t % kPfGroup == 0) {
      // this wave's loads of the group landed ...
      if (t == 0) wait_vmcnt<2 * kDmaPerWave * (kStages - kPfGroup)>();
      else wait_vmcnt<2 * kDmaPerWave * (kStages - 2 * kPfGroup)>();
      __builtin_amdgcn_s_barrier();  // ... and every wave's
    }
    if (load_here && t + kAhead >= kStages) issue(t + kAhead);
  };
  int t = 0;
  if (w_tiles > 1) {
    sync(0, false);
    qk(0);
    first_softmax(0, F_{});
    pv(0);
    t = 1;
  }
  for (; t + 1 < w_tiles; ++t) {
    sync(t, false);
    qk(t);
    stale_softmax(t, F_{});
    pv(t);
  }
  if (t + 1 == w_tiles) {  // the wave's last tile, masked
    sync(t, false);
    qk(t);
    if (t == 0) first_softmax(t, T_{});
    else stale_softmax(t, T_{});
    pv(t);
    ++t;
  }
  for (; t < n_tiles; ++t) sync(t, true);
  wait_vmcnt<0>();  // no load may still target this workgroup's LDS when it exits
  acc_gap();

  const float l_tot = pair32_sum(l_run);
  const float inv = (l_tot > 0.f) ? 1.f / l_tot : 0.f;
  if (Lse && hl == 0 && myq >= 0 && myq < S)
    Lse[(size_t)(b * Hq + h) * S + myq] = row_lse(m_run, l_tot);
  if (myq >= 0 && myq < S) {
#pragma unroll
    for (int ob = 0; ob < kNOB; ++ob) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d = 32 * ob + 8 * a + 4 * hl;
        const vec2 lo = Tr::pack2(o[ob][4 * a] * inv, o[ob][4 * a + 1] * inv);
        const vec2 hi = Tr::pack2(o[ob][4 * a + 2] * inv, o[ob][4 * a + 3] * inv);
        vec4 w;
        w[0] = lo[0]; w[1] = lo[1]; w[2] = hi[0]; w[3] = hi[1];
        *(vec4*)(Op + (size_t)myq * D + d) = w;
      }
    }
  }
}

template <typename Tr, int D, bool CAUSAL, bool POS>
__global__ __launch_bounds__(64 * kPfWaves, 1) void prefill_dma_kernel(
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
    prefill_dma_qtile<Tr, D, CAUSAL, POS>(Q, K, V, O, Lse, S, Hq, Hkv, scale_log2,
                                          pass ? wk.bh1 : wk.bh0, pass ? wk.qt1 : wk.qt0, q_shift, rq);
  }
}

template <typename Tr, int D, bool CAUSAL>
static hipError_t launch_prefill_dma(const void* q, const void* k, const void* v, void* o, float* lse,
                                     int B, int Hq, int Hkv, int S, float scale,
                                     hipStream_t stream, RopeQ rq) {
  using Gm = PfGeom<D>;
  static_assert(kPfStages * Gm::kStageB <= 160 * 1024, "LDS ring");
  const int n_qt = (S + kPfRows - 1) / kPfRows;
  // the padding rows of a ragged S go before row 0, in whole key tiles (so a
  // wave's causal diagonal still lies in one key tile): the partial tile is
  // the first one, whose causal key walk is the shortest
  const int q_shift = (n_qt * kPfRows - S) / Gm::kBN * Gm::kBN;
  int paired = 0;
  const long long grid = prefill_grid(B, Hq, n_qt, CAUSAL, 1, &paired);
  if (grid == 0) return hipSuccess;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  const float sl2 = scale * kLog2e;
  const dim3 block(64 * kPfWaves);
  if (sl2 >= 0.f) {
    hipLaunchKernelGGL((prefill_dma_kernel<Tr, D, CAUSAL, true>), dim3((unsigned)grid), block, 0,
                       stream, (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,
                       (uint16_t*)o, lse, S, Hq, Hkv, sl2, n_qt, B * Hq, (int)grid, paired, q_shift,
                       rq);
  } else {
    hipLaunchKernelGGL((prefill_dma_kernel<Tr, D, CAUSAL, false>), dim3((unsigned)grid), block, 0,
                       stream, (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,
                       (uint16_t*)o, lse, S, Hq, Hkv, sl2, n_qt, B * Hq, (int)grid, paired, q_shift,
                       rq);
  }
  return hipGetLastError();
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
