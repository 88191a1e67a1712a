// Prefill (flash-attention forward) for gfx950: bf16/fp16 MFMA, K/V tiles in
// LDS, online softmax in registers.
//
// Computes O = softmax(Q K^T * scale [+ causal mask]) V per (batch, q-head),
// the contract of dispatch_flash_attention_v2 / _v3_hopper / fused_gqa in the
// reference (kernels_api.h:29-33,52-56,78-83; math flash_attention_v2_kernel.cuh:
// 82-83 causal tile bound, 179-229 online softmax, 223 l == 0 -> 0).
//
// Work decomposition
//   one query tile = 256 query rows of one (b, h), taken by 8 waves; a
//   workgroup takes one query tile, a causal pair of them, or (persistent
//   launch, one workgroup per CU) every grid-th such item in turn;
//   each wave owns 32 query rows for the whole KV walk;
//   KV tiles of 64 keys travel HBM -> LDS by buffer loads into a ring of 4
//   tiles (8 at head dim 64) shared by the 8 waves; the two waves of a SIMD
//   run the ping-pong walk (16-bit head dim 128: one waits at the per-tile
//   barrier before its MFMA block, the other after it, so one's softmax runs
//   under the other's MFMAs) or the lockstep walk (head dim 64: one barrier
//   per four tiles).
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
// every K and V tile). Tile layout: 64 rows x 2D bytes,
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
constexpr int kPfStages = 4;   // K/V tiles in the LDS ring (32 KB each at D = 128; D = 64: 8)
constexpr int kPfKDepth = 1;   // K fragments read ahead of the QK MFMAs (k-steps)
constexpr int kPfVDepth = 2;   // V^T fragments read ahead of the PV MFMAs (steps)
// Key tiles per workgroup barrier of the lockstep walk: one barrier every
// two tiles lets a SIMD's two waves drift apart within the pair instead of
// meeting after every PV (+1.5 % over one barrier per tile on the 16-bit
// walk then in use). Head dim 64, whose 16 KB tiles
// let the ring hold eight, takes a barrier every four (+1.7 to +2.4 % on
// the reference grid's fp16 shapes).
constexpr int kPfGroup = 2;
constexpr int pf_stages(int d) { return d == 64 ? 8 : kPfStages; }
constexpr int pf_group(int d) { return d == 64 ? 4 : kPfGroup; }
// Ping-pong walk: tile t + kPpAhead is loaded with tile t (its slot held
// tile t - 2, released by the barrier of tile t).
constexpr int kPpAhead = 2;
// 24 wait states: longer than any MFMA-result -> VALU and VALU -> MFMA-operand
// hazard of gfx950, so MFMAs issued before it have written their results.
__device__ __forceinline__ void acc_gap() { CA_DEVICE_ASM("s_nop 7\n\ts_nop 7\n\ts_nop 7"); }

// A query tile of a workgroup: 256 rows of head bh (qt < 0: none).
struct PfItem {
  int bh, qt;
};

// One query tile (256 rows of head bh) of the workgroup: the whole key walk
// and the output store. Per wave and KV tile: QK (16 MFMAs at D = 128), the
// softmax step, PV (16 MFMAs); the overlap of MFMA and VALU comes from the
// other wave on the SIMD. MFMA blocks run at raised wave priority
// (s_setprio), so a wave's MFMAs win issue over its partner wave's softmax
// VALU.
//
// A workgroup takes its tiles one after another, and the ring keeps
// streaming across them: ring tiles are numbered from g0 (the tiles of the
// earlier items), and in the ping-pong walk the two loads past this item's
// last key tile fetch the first two key tiles of the next item `nx` instead
// of zeros; its Q rows are loaded before this item's output store. The
// return value says so (`pre` of the next call: its first tiles and Q rows
// are in flight). Otherwise (lockstep walk, no next item, or a walk shorter
// than kPpAhead tiles) every wave has waited for its own loads on return,
// other waves may still read the ring, and the caller puts a barrier before
// the next item.
//
template <typename Tr, int D, bool CAUSAL, bool POS>
__device__ CA_INLINE bool prefill_dma_qtile(const void* __restrict__ Qv, const void* __restrict__ Kv,
                                            const uint16_t* __restrict__ V, void* __restrict__ Ov,
                                            float* __restrict__ Lse, int S, int Hq, int Hkv, float scale_log2,
                                            int bh, int qt, int q_shift, RopeQ rq, PfItem nx, bool pre,
                                            int& g0, typename Tr::vec8 (&qv)[D / 16]) {
  using Gv = PfGeom<D>;                   // K and V tile geometry
  using Gk = Gv;
  using vec8 = typename Tr::vec8;
  using ovec4 = typename Tr::vec4;
  using ovec2 = typename Tr::vec2;
  constexpr int kBN = Gv::kBN;
  constexpr int kKRowB = Gk::kRowB, kVRowB = Gv::kRowB;       // bytes per K / V row in LDS
  constexpr int kKTileB = kBN * kKRowB, kVTileB = kBN * kVRowB;
  constexpr int kStageB = kKTileB + kVTileB;
  constexpr int kNOB = Gv::kNOB;
  constexpr int kBM = kPfRows, kStages = pf_stages(D), kNW = kPfWaves;
  constexpr int kGroup = pf_group(D);
  constexpr int kKL = kKTileB / 1024 / kNW;  // 1 KB K loads per wave per tile
  constexpr int kVL = kVTileB / 1024 / kNW;  // 1 KB V loads per wave per tile
  constexpr int kLoads = kKL + kVL;
  static_assert(kKL >= 1 && kVL >= 1 && kKTileB % (1024 * kNW) == 0 && kVTileB % (1024 * kNW) == 0,
                "tile loads");
  static_assert(kStageB % 256 == 0, "stage alignment (bank rows)");
  // QK steps (MFMAs issued after one K fragment wait): k-steps of 16 d
  constexpr int kQkSteps = Gv::kNKS;
  // The ping-pong walk (below) for head dim 128: same-box C2 +6.6 %, C2'
  // +4.9 %; at head dim 64 (-5 to -7 %) the MFMA blocks are too short to
  // hide the partner's softmax and the lockstep walk stays.
  constexpr bool kPingPong = D == 128;
  static_assert(kQkSteps % kLoads == 0, "loads spread over the QK steps");
  static_assert((kStages & (kStages - 1)) == 0, "ring slots: tile & (kStages - 1)");

  __shared__ __attribute__((aligned(1024))) unsigned char lds[kStages * kStageB];
  // per wave: 32 output rows x 128 bytes, staging the output store
  constexpr int kOStgB = 32 * 128;
  __shared__ __attribute__((aligned(16))) unsigned char ostg[kNW * kOStgB];

  // the K (V) rows of head bh's kv head
  auto kv_rows = [&](int bx) CA_INLINE {
    const int hx = bx % Hq;
    return (size_t)((bx / Hq) * Hkv + hx / (Hq / Hkv)) * S;
  };
  const int q0 = qt * kBM - q_shift;  // tile 0 may start before row 0 (rows < 0 are padding)
  const size_t qhead = (size_t)bh * S, khead = kv_rows(bh);
  const unsigned char* Kp = (const unsigned char*)Kv + khead * kKRowB;
  const uint16_t* Vp = V + khead * D;

  const int lane = __builtin_amdgcn_workitem_id_x() & 63;
  const int wave = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_workitem_id_x() >> 6);
  const int l32 = lane & 31, hl = lane >> 5;
  const int qw0 = q0 + wave * 32;
  const int myq = qw0 + l32;
  const bool q_in = myq >= 0 && myq < S;

  // Q as the B operand of S^T = K Q^T: qv, k-step ks: d = 16 ks + 8 hl +
  // [0, 8). Loaded after the first K/V tiles' loads, so that
  // their latencies overlap: the lane's row of tile (bx, qtx), row 0 for
  // rows outside [0, S) ...
  auto load_q_raw = [&](int bx, int qtx) CA_INLINE {
    const int r = qtx * kBM - q_shift + wave * 32 + l32;
    const size_t row = (size_t)bx * S + ((r >= 0 && r < S) ? r : 0);
    const uint16_t* Qr = (const uint16_t*)Qv + row * D;
#pragma unroll
    for (int ks = 0; ks < Gv::kNKS; ++ks) qv[ks] = *(const vec8*)(Qr + 16 * ks + 8 * hl);
  };
  // ... then zeroed outside [0, S) and rotated (RoPE).
  auto fix_q = [&]() CA_INLINE {
    if (!q_in) {
#pragma unroll
      for (int ks = 0; ks < Gv::kNKS; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[ks][e] = 0;
    }
    if (rq.cos && q_in) rope_q<Tr, D>(qv, rq, myq, hl);
  };

  const int kv_end = CAUSAL ? min(S, q0 + kBM) : S;
  const int n_tiles = (kv_end + kBN - 1) / kBN;
  // The next item's first kPpAhead key tiles take the ring places of this
  // item's tiles n_tiles .. n_tiles + kPpAhead - 1 (ping-pong walk, when this
  // walk is at least that long: its own first tiles are then all real).
  const bool redir = kPingPong && nx.qt >= 0 && n_tiles >= kPpAhead;
  const size_t khead_n = kv_rows(nx.bh);
  const unsigned char* Kp_n = (const unsigned char*)Kv + khead_n * kKRowB;
  const uint16_t* Vp_n = V + khead_n * D;
  const int kv_end_n = CAUSAL ? min(S, nx.qt * kBM - q_shift + kBM) : S;
  // tiles this wave computes on (it still loads and synchronises for all)
  const int w_end = CAUSAL ? min(kv_end, qw0 + 32) : kv_end;
  const int w_tiles = (qw0 + 32 > 0 && qw0 < S) ? (w_end + kBN - 1) / kBN : 0;

  // HBM -> LDS with buffer loads over the keys this workgroup needs
  // ([0, kv_end) of the (b, kv head) slice; rows past it read as zero, so
  // partial and trailing tiles need no clamp). K load i of this wave covers
  // tile rows kRpk*(kKL*wave + i) + lane/kLpr (likewise V); the lane fetches
  // the chunk that belongs at position lane % kLpr. Tile tt reads through
  // resources that start at its first row.
  uint32_t k_off[kKL], v_off[kVL];
#pragma unroll
  for (int i = 0; i < kKL; ++i) {
    const int row = Gk::kRpk * (kKL * wave + i) + lane / Gk::kLpr;
    k_off[i] = row * kKRowB + 16 * ((lane % Gk::kLpr) ^ Gk::swz(row));
  }
#pragma unroll
  for (int i = 0; i < kVL; ++i) {
    const int row = Gv::kRpk * (kVL * wave + i) + lane / Gv::kLpr;
    v_off[i] = row * kVRowB + 16 * ((lane % Gv::kLpr) ^ Gv::swz(row));
  }
  // load j of tile tt: K loads, then V loads.
  // Ring slot (g0 + tt) mod kStages; past this item's last tile, the next
  // item's tile tt - n_tiles when redirected (else rows past kv_end: zeros).
  auto issue_one = [&](int tt, int j) CA_INLINE {
    unsigned char* st = lds + ((g0 + tt) & (kStages - 1)) * kStageB;
    const bool o = redir && tt >= n_tiles;
    const uint32_t lt = (uint32_t)(o ? tt - n_tiles : tt);
    const uint32_t end = (uint32_t)(o ? kv_end_n : kv_end);
    if (j < kKL) {
      dma16_buf(make_rsrc_at(o ? Kp_n : Kp, lt * kKTileB, end * kKRowB),
                (CA_LDS void*)(st + 1024 * (kKL * wave + j)), k_off[j]);
    } else {
      const int i = j - kKL;
      dma16_buf(make_rsrc_at(o ? Vp_n : Vp, lt * kVTileB, end * kVRowB),
                (CA_LDS void*)(st + kKTileB + 1024 * (kVL * wave + i)), v_off[i]);
    }
  };
  auto issue = [&](int tt) CA_INLINE {
#pragma unroll
    for (int j = 0; j < kLoads; ++j) issue_one(tt, j);
  };

  // LDS read addresses (bytes from the stage base).
  // K: lane reads row krow (+32 per key block), logical chunk 2*ks + hl.
  const int krow = (l32 & 0x13) | ((l32 & 4) << 1) | ((l32 & 8) >> 1);
  const int fk = Gk::swz(krow);
  const uint32_t kofs = krow * kKRowB + 32 * (fk >> 1) + 16 * (hl ^ (fk & 1));  // ^ 32*ks
  // V^T: tr16 source lane -> row tr_row (+4 for the second read), logical
  // chunk 4*ob + c0, byte 8*(s16 & 1) of it.
  const int g16 = lane >> 4, s16 = lane & 15;
  const int tr_row = 8 * (g16 >> 1) + (s16 >> 2);
  const int c0 = 2 * (g16 & 1) + ((s16 & 3) >> 1);
  // D = 128: swz(tr_row + 4) == swz(tr_row) + 1 (tr_row % 8 < 4)
  const int fv = Gv::swz(tr_row);
  const int fv2 = D == 128 ? fv + 1 : Gv::swz(tr_row + 4);
  const uint32_t vofs1 = kKTileB + tr_row * kVRowB + 64 * (fv >> 2) + 16 * (c0 ^ (fv & 3)) + 8 * (s16 & 1);
  const uint32_t vofs2 =
      kKTileB + (tr_row + 4) * kVRowB + 64 * (fv2 >> 2) + 16 * (c0 ^ (fv2 & 3)) + 8 * (s16 & 1);
  const uint32_t lds0 = lds_off(lds);
  auto stage = [&](int tt) CA_INLINE {
    return lds0 + (uint32_t)(((g0 + tt) & (kStages - 1)) * kStageB);
  };

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
  // with j = p%4; sv[8kk + e] <-> P^T k-step kk); two partial row sums.
  // On a masked tile a masked logit gets weight 0 directly: its exponent
  // kMaskVal * scale_log2 - msub is -inf for every nonzero scale, but NaN for
  // scale 0 (softmax_scale = 0: equal weights for the visible keys).
  float psum[2];
  auto exp_pair = [&](int p, auto mask_tag) CA_INLINE {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int kk = p >> 2, j = p & 3;
    const int i0 = 8 * kk + 2 * j;
    float p0 = fast_exp2(__builtin_fmaf(sv[i0], scale_log2, -msub));
    float p1 = fast_exp2(__builtin_fmaf(sv[i0 + 1], scale_log2, -msub));
    if constexpr (MASK) {
      p0 = sv[i0] == kMaskVal ? 0.f : p0;
      p1 = sv[i0 + 1] == kMaskVal ? 0.f : p1;
    }
    const typename Tr::vec2 pk = Tr::pack2(p0, p1);
    pb[kk][2 * j] = pk[0];
    pb[kk][2 * j + 1] = pk[1];
    // pairs 0 and 1 start the two chains
    psum[j & 1] = p < 2 ? p0 + p1 : psum[j & 1] + (p0 + p1);
  };
  auto exp_all = [&](auto mask_tag) CA_INLINE {
#pragma unroll
    for (int p = 0; p < 16; ++p) exp_pair(p, mask_tag);
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
    // a row all masked in this tile has no max (also for scale 0)
    const float tmax = pair32_max(t2 == kMaskVal ? kNegInf : t2 * scale_log2);
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
    exp_all(mask_tag);
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
    exp_all(mask_tag);
    if (__builtin_expect(wave_any(!(psum[0] + psum[1] <= kStaleMax)), 0)) {
      tm[0] = tm[1] = kMaskVal;
#pragma unroll
      for (int p = 0; p < 16; ++p) fold_max(p);
      settle_max();
      exp_all(mask_tag);
    }
    l_run += psum[0] + psum[1];
  };

  // S^T(tn) = K(tn) Q^T, K fragments kPfKDepth steps ahead of the MFMAs.
  // The wave's loads of tile tn + kStages - kGroup go out between its QK
  // steps, one after every kQkSteps / kLoads of them: issued all at once
  // after the barrier, the 8 waves' loads queue behind each other (C2
  // +1.8 %).
  constexpr int kAhead = kStages - kGroup;
  static_assert(kAhead >= kGroup, "a barrier group's tiles are issued before its barrier");
  auto qk = [&](int tn) CA_INLINE {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[mb][r] = 0.f;
    __builtin_amdgcn_s_setprio(1);
    const uint32_t ka = stage(tn) + kofs;
    constexpr int KD = kPfKDepth;
    u32x4 kr[KD + 1][2];
    // step st's K fragment: k-step st of both key blocks
    auto kread = [&](int st) CA_INLINE {
      const uint32_t an = ka ^ (32 * st);
      kr[st % (KD + 1)][0] = lds_read_b128<0>(an);
      kr[st % (KD + 1)][1] = lds_read_b128<32 * kKRowB>(an);
    };
#pragma unroll
    for (int st = 0; st < KD; ++st) kread(st);
#pragma unroll
    for (int st = 0; st < kQkSteps; ++st) {
      const int cb = st % (KD + 1);
      if (st + KD < kQkSteps) kread(st + KD);
      wait_lgkm_n(2 * (KD < kQkSteps - 1 - st ? KD : kQkSteps - 1 - st));  // step st landed
      after_wait(kr[cb][0]);
      after_wait(kr[cb][1]);
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        sacc[mb] = Tr::mfma32(__builtin_bit_cast(vec8, kr[cb][mb]), qv[st], sacc[mb]);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);  // then up to 8 VALU
      }
      if (st % (kQkSteps / kLoads) == kQkSteps / kLoads - 1)
        issue_one(tn + kAhead, st / (kQkSteps / kLoads));
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
    constexpr int NST = 4 * kNOB;     // steps: kNOB O^T blocks x 4 P^T k-steps
    constexpr int kKK = 16 * kVRowB;  // bytes per P^T k-step of V rows
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

  // ---- MFMA block M(s) = PV(s-1) then QK(s) --------------------------------
  // One MFMA per step: PV steps (O^T block i / 4, P^T k-step i % 4; V^T
  // fragment = two tr16 reads) then QK steps (key block j % 2, k-step j / 2;
  // K fragment = one b128 read). Fragments stream kMD steps
  // ahead across the PV -> QK boundary, so a wave keeps the matrix pipe fed
  // on its own while its partner runs the softmax. The loads of tile s +
  // kAhead go out between the QK steps.
  constexpr int kNPV = 4 * kNOB;
  constexpr int kNQK = 2 * Gv::kNKS;
  constexpr int kRQK = 1;           // LDS reads per QK step
  constexpr int kMD = 4;            // steps read ahead
  static_assert(kNQK % kLoads == 0, "loads spread over the QK steps");
  constexpr int kKK = 16 * kVRowB;  // bytes per P^T k-step of V rows
  // A wave's LDS reads run at ~1 KB per 35-40 cycles, slower than its MFMAs
  // consume them, and its softmax block issues none: the V^T fragments of
  // the first kNPF PV steps of M(s + 1) are read during softmax(s) (tile s
  // is resident from barrier s until barrier s + 2, which follows M(s + 1)).
  constexpr int kNPF = 4;
  u32x4 pvf[kNPF];
  auto pv_read = [&](uint32_t va1, uint32_t va2, int i) CA_INLINE {
    const uint32_t x = 64 * (i >> 2);
    u32x2 a, c;
    switch (i & 3) {
      case 0: a = lds_read_tr16<0>(va1 ^ x); c = lds_read_tr16<0>(va2 ^ x); break;
      case 1: a = lds_read_tr16<kKK>(va1 ^ x); c = lds_read_tr16<kKK>(va2 ^ x); break;
      case 2: a = lds_read_tr16<2 * kKK>(va1 ^ x); c = lds_read_tr16<2 * kKK>(va2 ^ x); break;
      default: a = lds_read_tr16<3 * kKK>(va1 ^ x); c = lds_read_tr16<3 * kKK>(va2 ^ x); break;
    }
    return u32x4{a[0], a[1], c[0], c[1]};
  };
  auto pv_prefetch = [&](int t) CA_INLINE {
    const uint32_t va1 = stage(t) + vofs1, va2 = stage(t) + vofs2;
#pragma unroll
    for (int i = 0; i < kNPF; ++i) pvf[i] = pv_read(va1, va2, i);
  };
  auto mblock = [&](int s, auto pv_tag, auto qk_tag) CA_INLINE {
    constexpr bool DPV = decltype(pv_tag)::value, DQK = decltype(qk_tag)::value;
    constexpr int NPV = DPV ? kNPV : 0, N = NPV + (DQK ? kNQK : 0);
    __builtin_amdgcn_s_setprio(1);
    const uint32_t va1 = stage(s + kStages - 1) + vofs1, va2 = stage(s + kStages - 1) + vofs2;
    const uint32_t ka = stage(s) + kofs;
    if constexpr (DQK) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[mb][r] = 0.f;
    }
    u32x4 fr[kMD + 1][kRQK];
    // steps [0, P0) take the fragments read during the softmax; the ring
    // streams steps [P0, N)
    constexpr int P0 = DPV ? kNPF : 0;
    auto nreads = [&](int i) CA_INLINE { return i < NPV ? 2 : kRQK; };
    auto fread = [&](int i) CA_INLINE {
      const int b = i % (kMD + 1);
      if (i < NPV) {
        fr[b][0] = pv_read(va1, va2, i);
      } else {
        const int j = i - NPV, mb = j & 1, ks = j >> 1;
        if (mb == 0) {
          fr[b][0] = lds_read_b128<0>(ka ^ (32 * ks));
        } else {
          fr[b][0] = lds_read_b128<32 * kKRowB>(ka ^ (32 * ks));
        }
      }
    };
#pragma unroll
    for (int i = P0; i < P0 + kMD && i < N; ++i) fread(i);
    if constexpr (P0 > 0) {
      int pending = 0;  // the ring reads just issued; the prefetched ones are older
#pragma unroll
      for (int k = P0; k < P0 + kMD && k < N; ++k) pending += nreads(k);
      wait_lgkm_n(pending);
#pragma unroll
      for (int i = 0; i < P0; ++i) after_wait(pvf[i]);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int b = i % (kMD + 1);
      if (i >= P0) {
        if (i + kMD < N) fread(i + kMD);
        int pending = 0;  // reads issued after step i's
#pragma unroll
        for (int k = i + 1; k <= i + kMD && k < N; ++k) pending += nreads(k);
        wait_lgkm_n(pending);
#pragma unroll
        for (int r = 0; r < kRQK; ++r) after_wait(fr[b][r]);
      }
      if (i < NPV) {
        const int ob = i >> 2, kk = i & 3;
        const u32x4 va = i < P0 ? pvf[i < P0 ? i : 0] : fr[b][0];
        o[ob] = Tr::mfma32(__builtin_bit_cast(vec8, va), pb[kk], o[ob]);
      } else {
        const int j = i - NPV, mb = j & 1, ks = j >> 1;
        sacc[mb] = Tr::mfma32(__builtin_bit_cast(vec8, fr[b][0]), qv[ks], sacc[mb]);
        if (j % (kNQK / kLoads) == kNQK / kLoads - 1) issue_one(s + kPpAhead, j / (kNQK / kLoads));
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // ---- the tile walk ----------------------------------------------------------
  // Every wave walks all n_tiles tiles (it loads its share of each and meets
  // the others at the barrier of every tile pair). Only a wave's last tile
  // can need a mask (bounds or causal diagonal); it is masked when taken out
  // of the accumulators. The wave's first tile takes the full row max, later
  // tiles the stale-max step.
  using T_ = std::true_type;
  using F_ = std::false_type;
  if constexpr (kPingPong) {
    // Ping-pong walk. Each wave alternates its MFMA block M(s) and its softmax
    // V(s); the waves of a SIMD (w and w + 4) run half a tile apart, so one
    // wave's softmax runs under the other's MFMAs: waves 0-3 meet the barrier
    // of tile t before M(t), waves 4-7 right after M(t - 1). Barrier t (every
    // tile): every wave has tile t resident (its own loads waited on, the
    // others' by the barrier) and is past its last read of tile t - 2 (PV(t -
    // 2) is in M(t - 1), before either placement), whose slot takes tile t +
    // 2, issued in M(t) or, for a wave with no QK(t), right after it. Before
    // every barrier a wave has issued tiles up to t + 1, so one tile's loads
    // may still be in flight.
    const bool lead = wave < 4;
    auto bar = [&](int t) CA_INLINE {
      if (t < n_tiles) {
        wait_vmcnt<kLoads>();
        __builtin_amdgcn_s_barrier();
      }
    };
    if (!pre) {  // else the previous item issued them
#pragma unroll
      for (int tt = 0; tt < kPpAhead; ++tt) issue(tt);
      load_q_raw(bh, qt);
    }
    fix_q();
    if (!lead) bar(0);
    int s = 0;
    if (w_tiles > 0) {
      // tile 0: QK only, the full row max
      if (lead) bar(0);
      mblock(0, F_{}, T_{});
      if (!lead) bar(1);
      pv_prefetch(0);
      if (w_tiles > 1) first_softmax(0, F_{});
      else first_softmax(0, T_{});
      // steady tiles: PV(s - 1) + QK(s), the stale-max softmax
      for (s = 1; s + 1 < w_tiles; ++s) {
        if (lead) bar(s);
        mblock(s, T_{}, T_{});
        if (!lead) bar(s + 1);
        pv_prefetch(s);
        stale_softmax(s, F_{});
      }
      if (s < w_tiles) {  // the wave's last tile, masked
        if (lead) bar(s);
        mblock(s, T_{}, T_{});
        if (!lead) bar(s + 1);
        pv_prefetch(s);
        stale_softmax(s, T_{});
        ++s;
      }
      // PV of the last tile
      if (lead) bar(s);
      mblock(s, T_{}, F_{});
      if (s < n_tiles) issue(s + kPpAhead);
      if (!lead) bar(s + 1);
    } else {
      if (lead) bar(0);
      issue(kPpAhead);
      if (!lead) bar(1);
    }
    int t = s + 1;  // w_tiles + 1: the walk met barriers 0 .. w_tiles (lead) or 0 .. w_tiles + 1
    if (!lead) {
      if (t < n_tiles) issue(t + kPpAhead);
      ++t;
    }
    for (; t < n_tiles; ++t) {
      bar(t);
      issue(t + kPpAhead);
    }
  } else {
    // Tiles 0 .. kAhead - 1 go out up front; tile t + kAhead with tile t: a
    // wave that computes on tile t issues its loads inside qk(t), one that
    // does not in sync(t, true), so the steady-state walk has no condition on
    // them. Tiles past the walk's end (short walks) read zeros into their
    // slots without a memory access.
#pragma unroll
    for (int tt = 0; tt < kAhead; ++tt) issue(tt);
    load_q_raw(bh, qt);
    fix_q();
    // Barrier at tile t (t % kGroup == 0): every wave has its loads of tiles
    // t .. t + kGroup - 1 resident and is past its last read of tile t - 1,
    // so the slots of tiles t - kGroup .. t - 1 take tiles t + kAhead ..
    // The wave has issued tiles up to t + kAhead - 1 by then, so the loads of
    // kAhead - kGroup tiles may still be in flight (kAhead >= kGroup: the
    // group's tiles were all issued before its barrier).
    auto sync = [&](int t, bool load_here) CA_INLINE {
      if (t % kGroup == 0) {
        wait_vmcnt<kLoads * (kAhead - kGroup)>();  // this wave's loads of the group landed ...
        __builtin_amdgcn_s_barrier();                // ... and every wave's
      }
      if (load_here) issue(t + kAhead);
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
  }
  // Unless the next item's first tiles are in flight into the ring, no load
  // may still target it when the next item drains it or the workgroup exits.
  if (!redir) wait_vmcnt<0>();
  acc_gap();
  if constexpr (kPingPong) {
    if (redir) load_q_raw(nx.bh, nx.qt);  // this item's Q is dead after its last QK
  }

  const float l_tot = pair32_sum(l_run);
  const float inv = (l_tot > 0.f) ? 1.f / l_tot : 0.f;
  if (Lse && hl == 0 && q_in) Lse[qhead + myq] = row_lse(m_run, l_tot);
  // The output rows go out through the wave's LDS block, 64 d (128 bytes)
  // of its 32 rows per pass: O^T spreads a row over two lanes, 4 d per
  // register group, so stores straight from registers would write 16 bytes
  // of 32 rows per instruction; from the block, each store instruction
  // writes 8 whole rows of the pass (8 full 128-byte lines). Block layout:
  // row r at 128 r, 16-byte chunk c at position c ^ (r % 8). A wave's LDS
  // accesses complete in order, so the passes need no barrier; they are
  // issued by hand, so that they need not wait for the next tile's K/V
  // loads into the ring.
  constexpr int kPassOb = 2;  // O^T blocks (32 d each) per pass
  const uint32_t ob_base = lds_off(ostg) + (uint32_t)(wave * kOStgB);
#pragma unroll
  for (int p = 0; p < kNOB / kPassOb; ++p) {
#pragma unroll
    for (int j = 0; j < kPassOb; ++j) {
      const int ob = kPassOb * p + j;
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const ovec2 lo = Tr::pack2(o[ob][4 * a] * inv, o[ob][4 * a + 1] * inv);
        const ovec2 hi = Tr::pack2(o[ob][4 * a + 2] * inv, o[ob][4 * a + 3] * inv);
        ovec4 w;
        w[0] = lo[0]; w[1] = lo[1]; w[2] = hi[0]; w[3] = hi[1];
        const int c = 4 * j + a;  // d = 64 p + 8 c + 4 hl + [0, 4)
        lds_write_b64<0>(ob_base + 128 * l32 + 16 * (c ^ (l32 & 7)) + 8 * hl,
                         __builtin_bit_cast(u32x2, w));
      }
    }
    u32x4 rows[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = 8 * k + (lane >> 3), c = lane & 7;
      rows[k] = lds_read_b128<0>(ob_base + 128 * r + 16 * (c ^ (r & 7)));
    }
    wait_lgkm<0>();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      after_wait(rows[k]);
      const int r = 8 * k + (lane >> 3), c = lane & 7;
      const int row = qw0 + r;
      if (row >= 0 && row < S) *(u32x4*)((uint16_t*)Ov + (qhead + row) * D + 64 * p + 8 * c) = rows[k];
    }
  }
  g0 += n_tiles;
  return redir;
}

// Operands of a prefill launch: Q, K, V 16-bit rows; O the output rows.
struct PfArgs {
  const void* q;
  const void* k;
  const uint16_t* v;
  void* o;
  float* lse;
};

template <typename Tr, int D, bool CAUSAL, bool POS>
__global__ __launch_bounds__(64 * kPfWaves, 1) void prefill_dma_kernel(
    PfArgs a, int S, int Hq, int Hkv, float scale_log2, int n_qt, int n_bh, int n_work, int paired,
    int q_shift, RopeQ rq) {
  // Work items v = blockIdx.x, + gridDim.x, ... (a persistent launch when the
  // grid is smaller than n_work; gridDim.x is then a multiple of 8, so every
  // item keeps the XCD that xcd_remap gives it). A paired item is two query
  // tiles; a pair's long tile runs first: the pair workgroups of a head then
  // start their walks together over the same keys and share their L2 lines
  // (short tile first measured slower on C2, with more HBM fetches).
  typename Tr::vec8 qv[D / 16];
  int g0 = 0;  // ring tiles taken by the earlier query tiles
  bool pre = false;
  int v = __builtin_amdgcn_workgroup_id_x(), pass = 0;
  QTileWork wk = prefill_work(xcd_remap(v, n_work), n_qt, n_bh, paired);
#pragma clang loop unroll(disable)
  for (;;) {
    // the tile after this one: the pair's second, else the next item's first
    int v2 = v, pass2 = pass + 1;
    QTileWork wk2 = wk;
    if (pass2 == 2 || wk.qt1 < 0) {
      v2 = v + (int)gridDim.x;
      pass2 = 0;
      if (v2 < n_work) wk2 = prefill_work(xcd_remap(v2, n_work), n_qt, n_bh, paired);
    }
    // Item indices and g0 are uniform; readfirstlane says so (else the
    // compiler may keep them in vector registers and wrap every buffer load
    // built from them in a loop over lanes).
    const int bh = __builtin_amdgcn_readfirstlane(pass ? wk.bh1 : wk.bh0);
    const int qt = __builtin_amdgcn_readfirstlane(pass ? wk.qt1 : wk.qt0);
    const PfItem nx0 = v2 < n_work ? PfItem{pass2 ? wk2.bh1 : wk2.bh0, pass2 ? wk2.qt1 : wk2.qt0}
                                   : PfItem{0, -1};
    const PfItem nx{__builtin_amdgcn_readfirstlane(nx0.bh), __builtin_amdgcn_readfirstlane(nx0.qt)};
    g0 = __builtin_amdgcn_readfirstlane(g0);
    pre = prefill_dma_qtile<Tr, D, CAUSAL, POS>(a.q, a.k, a.v, a.o, a.lse, S, Hq, Hkv, scale_log2, bh, qt,
                                                 q_shift, rq, nx, pre, g0, qv);
    if (nx.qt < 0) break;
    // a drained ring is refilled by the next tile: every wave must be done reading it
    if (!pre) __builtin_amdgcn_s_barrier();
    v = v2;
    pass = pass2;
    wk = wk2;
  }
}

// Grid, ragged-S shift and launch of the prefill kernel.
template <typename Tr, int D, bool CAUSAL>
static hipError_t launch_prefill_kernel(const PfArgs& a, int B, int Hq, int Hkv, int S, float scale,
                                        hipStream_t stream, RopeQ rq) {
  using Gm = PfGeom<D>;
  const int n_qt = (S + kPfRows - 1) / kPfRows;
  // the padding rows of a ragged S go before row 0, in whole key tiles (so a
  // wave's causal diagonal still lies in one key tile): the partial tile is
  // the first one, whose causal key walk is the shortest
  const int q_shift = (n_qt * kPfRows - S) / Gm::kBN * Gm::kBN;
  int paired = 0;
  const long long n_work = prefill_grid(B, Hq, n_qt, CAUSAL, 1, &paired);
  if (n_work == 0) return hipSuccess;
  if (n_work > 0x7fffffffLL) return hipErrorInvalidValue;
  // Items of equal work (non-causal tiles, causal pairs): one workgroup per
  // CU (the ring's LDS admits one) takes items v, v + grid, ..., so a
  // workgroup's next tile streams into the ring behind its current one.
  // Unpaired causal tiles differ in length and keep one workgroup each,
  // longest first, for the hardware dispatcher to balance.
  const long long slots = device_cus() / 8 * 8;
  const long long grid = ((!CAUSAL || paired) && slots > 0 && n_work > slots) ? slots : n_work;
  const float sl2 = scale * kLog2e;
  const dim3 block(64 * kPfWaves);
  if (sl2 >= 0.f) {
    hipLaunchKernelGGL((prefill_dma_kernel<Tr, D, CAUSAL, true>), dim3((unsigned)grid),
                       block, 0, stream, a, S, Hq, Hkv, sl2, n_qt, B * Hq, (int)n_work, paired,
                       q_shift, rq);
  } else {
    hipLaunchKernelGGL((prefill_dma_kernel<Tr, D, CAUSAL, false>), dim3((unsigned)grid),
                       block, 0, stream, a, S, Hq, Hkv, sl2, n_qt, B * Hq, (int)n_work, paired,
                       q_shift, rq);
  }
  return hipGetLastError();
}

template <typename Tr, int D, bool CAUSAL>
static hipError_t launch_prefill_dma(const void* q, const void* k, const void* v, void* o, float* lse,
                                     int B, int Hq, int Hkv, int S, float scale,
                                     hipStream_t stream, RopeQ rq) {
  const PfArgs a{q, k, (const uint16_t*)v, o, lse};
  return launch_prefill_kernel<Tr, D, CAUSAL>(a, B, Hq, Hkv, S, scale, stream, rq);
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
  if ((dtype == kDtypeBF16 || dtype == kDtypeF16) && prefill_w64_supported(D, S, scale, rq.cos != nullptr))
    return launch_prefill_w64(dtype == kDtypeF16, q, k, v, o, lse, B, Hq, Hkv, S, scale, causal, stream);
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
