// Flash-attention backward for gfx950 (bf16/fp16 MFMA, fp32 accumulation).
//
// Computes dQ, dK, dV of O = softmax(Q K^T * scale [+ causal mask]) V from Q,
// K, V, O, dO and the forward's natural-log row logsumexp LSE: the contract
// of dispatch_flash_attention_v2_backward (kernels_api.h:65-69), math of
// flash_attention_bwd_kernel.cuh:9-19 and 96-214:
//   D_i = rowsum(dO * O),  P = exp(S * scale - LSE_i),  dP = dO V^T,
//   dS = P (dP - D_i) * scale,  dQ = dS K,  dK = dS^T Q,  dV = P^T dO,
// with P = dS = 0 for masked entries (key > query when causal) and for keys
// or queries past S. GQA (Hkv < Hq, kv head = h / (Hq / Hkv)): dK and dV of a
// kv head are summed over its q heads.
//
// Three launches and no atomics, so the result does not depend on timing:
//   bwd_rowdot_kernel   the pair (LSE log2 e, D = rowsum(dO * O)) per query
//                       row into a [B, Hq, S] x 2 fp32 workspace;
//   bwd_dkv_dma_kernel  key-outer: 8 waves x 32 keys of one (b, kv head);
//                       query tiles of 32 (Q, dO, pairs) stream through an
//                       LDS ring, for every q head of the kv head; per tile
//                       S = Q K^T, dP = dO V^T, dS, dV^T += dO^T P,
//                       dK^T += Q^T dS;
//   bwd_dq_dma_kernel   query-outer: 8 waves x 32 queries of one (b, h); key
//                       tiles of 64 (K, V) stream through an LDS ring; per
//                       32 keys S^T = K Q^T, dP^T = V dO^T, dS^T,
//                       dQ^T += K^T dS^T.
// Operand layouts are those of the forward kernels (prefill.hip): the 32-row
// A operand of the first product of a tile reads its rows in the order
// rho(i) = i with bits 2 and 3 swapped, which puts row 16 (r/8) + 8 h + r%8
// into accumulator register r of lane half h. Those 8-register runs are
// exactly the 16-bit B operand (dV^T, dK^T, forward PV) or A operand (dQ) of
// the next product's k-steps, so P and dS go from accumulators to operands
// without leaving registers. The transposed operands (K^T, Q^T, dO^T) come
// from row-major LDS tiles through ds_read_b64_tr_b16.
#include "common.h"
#include "launch.h"
#include "lds_dma.h"

namespace ca {
namespace {

__device__ __forceinline__ int rho32(int i) { return (i & 0x13) | ((i & 4) << 1) | ((i & 8) >> 1); }

// Per query row of B * Hq * S: the pair (LSE * log2(e), D) with D = sum_d
// dO[row][d] * O[row][d] (flash_attention_bwd_kernel.cuh:96-108), so the
// kernels below fetch both terms of a row with one 8-byte load. D / 8 lanes
// per row, 8 elements each.
template <typename Tr, int D>
__global__ __launch_bounds__(256) void bwd_rowdot_kernel(const uint16_t* __restrict__ O,
                                                         const uint16_t* __restrict__ dO,
                                                         const float* __restrict__ LSE,
                                                         float* __restrict__ LD, long long rows) {
  using vec8 = typename Tr::vec8;
  constexpr int L = D / 8;
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long row = t / L;
  const int c = (int)(t % L);
  float acc = 0.f;
  if (row < rows) {
    const vec8 o = *(const vec8*)(O + row * D + 8 * c);
    const vec8 g = *(const vec8*)(dO + row * D + 8 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = __builtin_fmaf((float)o[e], (float)g[e], acc);
  }
#pragma unroll
  for (int m = L / 2; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if (row < rows && c == 0) {
    LD[2 * row] = LSE[row] * kLog2e;
    LD[2 * row + 1] = acc;
  }
}

// Store the transposed accumulators acc[ob] (lane (l32, hl) holds d = 32 ob +
// 8 a + 4 hl + [0, 4) of row l32) as the wave's 32 rows row0 + l32 (rows
// outside [0, n) skipped) of the [.., D] tensor at `head`, through the wave's
// LDS block at byte offset `stg` (32 rows x RB bytes, RB / 2 d per pass; row
// r's 16-byte chunk c at position c ^ (r % (RB / 16))). Stored from
// registers, a row's d are spread over two lanes, so every store instruction
// would write 16 bytes of 32 rows; from the block, each writes 64 / (RB / 16)
// whole RB-byte row pieces. The LDS accesses are hand-issued and in wave
// order, so the passes need no barrier.
template <typename Tr, int NOB, int RB>
__device__ __forceinline__ void store_rowsT_lds(uint16_t* head, int row0, int n,
                                                const f32x16 (&acc)[NOB], float mul, uint32_t stg,
                                                int lane) {
  using vec4 = typename Tr::vec4;
  using vec2 = typename Tr::vec2;
  constexpr int D = 32 * NOB;
  constexpr int NCH = RB / 16;   // 16-byte chunks per staged row
  constexpr int OBP = RB / 64;   // accumulator blocks (32 d) per pass
  constexpr int RPI = 64 / NCH;  // rows per LDS read / store instruction
  static_assert(NOB % OBP == 0 && 32 % RPI == 0, "store passes");
  const int l32 = lane & 31, hl = lane >> 5;
#pragma unroll
  for (int p = 0; p < NOB / OBP; ++p) {
#pragma unroll
    for (int j = 0; j < OBP; ++j) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int ob = OBP * p + j, c = 4 * j + a;  // d = 32 ob + 8 a + 4 hl + [0, 4)
        const vec2 lo = Tr::pack2(acc[ob][4 * a] * mul, acc[ob][4 * a + 1] * mul);
        const vec2 hi = Tr::pack2(acc[ob][4 * a + 2] * mul, acc[ob][4 * a + 3] * mul);
        vec4 w;
        w[0] = lo[0]; w[1] = lo[1]; w[2] = hi[0]; w[3] = hi[1];
        lds_write_b64<0>(stg + RB * l32 + 16 * (c ^ (l32 % NCH)) + 8 * hl,
                         __builtin_bit_cast(u32x2, w));
      }
    }
    u32x4 t[32 / RPI];
#pragma unroll
    for (int k = 0; k < 32 / RPI; ++k) {
      const int r = RPI * k + lane / NCH, c = lane % NCH;
      t[k] = lds_read_b128<0>(stg + RB * r + 16 * (c ^ (r % NCH)));
    }
    wait_lgkm<0>();
#pragma unroll
    for (int k = 0; k < 32 / RPI; ++k) {
      after_wait(t[k]);
      const int r = RPI * k + lane / NCH, c = lane % NCH;
      const int row = row0 + r;
      if (row >= 0 && row < n) *(u32x4*)(head + (size_t)row * D + (RB / 2) * p + 8 * c) = t[k];
    }
  }
}

// ---------------------------------------------------------------------------
// HBM -> LDS buffer-load kernels (head dim 64 and 128), 8 waves (two per SIMD)
// per workgroup.
//
// Tiles are rows of 2 D bytes stored unpadded, the 16-byte chunk c of row r
// at position c ^ swz(r), with swz chosen so that both read patterns are
// bank-conflict free: row reads (ds_read_b128, one chunk of 16 consecutive
// rows per 16 lanes; the A operand of S^T / S and dP^T / dP, and the V^T B
// operand of dP) and transposed reads (ds_read_b64_tr_b16, 4 chunks of 4
// consecutive rows per 32 lanes; the K^T, Q^T and dO^T A operands).
//   D = 128 (256-byte rows, the layout of the forward kernel):
//     swz(r) = 4 (r % 4) + (r / 4) % 4;
//   D = 64 (128-byte rows, two rows per 256 bytes of banks):
//     swz(r) = 4 ((r / 2) % 2) + (r / 4) % 4, which gives the 8 rows of one
//     parity among 16 consecutive rows 8 distinct chunks, and rows r and r + 2
//     opposite 4-chunk halves.
// 1/scale is folded out of dS and applied once when dQ and dK are stored.
// ---------------------------------------------------------------------------
namespace bwdma {
constexpr int kNW = 8;         // waves per workgroup
constexpr int kStages = 4;     // ring tiles
constexpr int kDist = kStages - 1;
struct TrOfs {
  uint32_t a, b;
};
template <int D>
struct Geom {
  static constexpr int kRowB = 2 * D;        // bytes per row
  static constexpr int kLpr = kRowB / 16;    // 16-byte chunks per row
  static constexpr int kRpk = 1024 / kRowB;  // rows per 1-KB load
  static constexpr int kNKS = D / 16;        // 16-deep k-steps over D
  static constexpr int kNOB = D / 32;        // 32-row blocks over D
  static_assert(D == 64 || D == 128, "head dim");
  __device__ static __forceinline__ int swz(int r) {
    return D == 128 ? (((r & 3) << 2) | ((r >> 2) & 3)) : ((((r >> 1) & 1) << 2) | ((r >> 2) & 3));
  }
  // Row-read byte offset: row `row`, logical chunk hl (XOR 32 * ks for chunk 2 ks + hl).
  __device__ static __forceinline__ uint32_t row_ofs(int row, int hl) {
    return row * kRowB + 16 * (hl ^ swz(row));
  }
  // Byte offset of the chunk a lane fetches in a 1-KB load whose first row is
  // `row0`: row row0 + lane / kLpr, logical chunk (lane % kLpr) ^ swz(row),
  // which lands at position lane % kLpr.
  __device__ static __forceinline__ uint32_t dma_ofs(int row0, int lane) {
    const int row = row0 + lane / kLpr;
    return row * kRowB + 16 * ((lane % kLpr) ^ swz(row));
  }
  // Transposed-read byte offsets of a lane (rows 8 (g16/2) + s16/4 and +4 of a
  // 16-row k-step, chunks 2 (g16 % 2) + (s16 % 4) / 2 of the 32 dims of a
  // block: XOR 64 ob for dims block ob), as in the forward's V^T reads.
  __device__ static __forceinline__ TrOfs tr_ofs(int lane) {
    const int g16 = lane >> 4, s16 = lane & 15;
    const int row = 8 * (g16 >> 1) + (s16 >> 2);
    const int c0 = 2 * (g16 & 1) + ((s16 & 3) >> 1);
    TrOfs t;
    t.a = row * kRowB + 16 * (c0 ^ swz(row)) + 8 * (s16 & 1);
    t.b = (row + 4) * kRowB + 16 * (c0 ^ swz(row + 4)) + 8 * (s16 & 1);
    return t;
  }
  // A operand (32 dims x 16 rows) of k-step kk of a tile at `base`, dims block ob.
  template <typename Tr, int KK>
  __device__ static __forceinline__ typename Tr::vec8 tr_operand(uint32_t base, TrOfs t, int ob) {
    const u32x2 lo = lds_read_tr16<16 * kRowB * KK>((base + t.a) ^ (64 * ob));
    const u32x2 hi = lds_read_tr16<16 * kRowB * KK>((base + t.b) ^ (64 * ob));
    const u32x4 w = {lo[0], lo[1], hi[0], hi[1]};
    return __builtin_bit_cast(typename Tr::vec8, w);
  }
};
}  // namespace bwdma

// dQ of query tile qt (256 rows) of head bh: the keys [0, kv_end) in tiles of
// 64, each computed as two halves of 32 keys.
template <typename Tr, int D, bool CAUSAL>
__device__ CA_INLINE void bwd_dq_dma_tile(const uint16_t* __restrict__ Q,
                                         const uint16_t* __restrict__ K,
                                         const uint16_t* __restrict__ V,
                                         const uint16_t* __restrict__ dO,
                                         const float* __restrict__ LD, uint16_t* __restrict__ dQ,
                                         int S, int Hq, int Hkv, float scale, int bh, int qt) {
  using namespace bwdma;
  using Gm = Geom<D>;
  using vec8 = typename Tr::vec8;
  using vec2 = typename Tr::vec2;
  constexpr int kRowB = Gm::kRowB, kNKS = Gm::kNKS, kNOB = Gm::kNOB;
  constexpr int BM = 32 * kNW;
  constexpr int BN = 64;
  constexpr int kTileB = BN * kRowB;           // 16 KB (D = 128), 8 KB (D = 64)
  constexpr int kStageB = 2 * kTileB;          // K tile, then V tile
  constexpr int kDma = kTileB / 1024 / kNW;    // 1-KB loads per wave per K (and V) tile
  static_assert(kDma * 1024 * kNW == kTileB, "whole 1-KB loads per wave");
  __shared__ __attribute__((aligned(1024))) unsigned char lds[kStages * kStageB];
  // per wave: 32 dQ rows x 128 bytes, staging the dQ store
  __shared__ __attribute__((aligned(16))) unsigned char qstg[kNW * 32 * 128];

  const int b = bh / Hq, h = bh % Hq;
  const int hk = h / (Hq / Hkv);
  const int q0 = qt * BM;
  const size_t qoff = (size_t)(b * Hq + h) * S;
  const uint16_t* Kp = K + (size_t)(b * Hkv + hk) * S * D;
  const uint16_t* Vp = V + (size_t)(b * Hkv + hk) * S * D;
  const int lane = __builtin_amdgcn_workitem_id_x() & 63;
  const int wave = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_workitem_id_x() >> 6);
  const int l32 = lane & 31, hl = lane >> 5;
  const int qw0 = q0 + 32 * wave;
  const int myq = qw0 + l32;
  const bool qvalid = myq < S;
  const float c2 = scale * kLog2e;
  float lse2 = -kNegInf, dd = 0.f;  // a query past S: P = 0
  vec8 qv[kNKS], gv[kNKS];          // Q and dO as B operands (column = this lane's query)
  if (qvalid) {
    lse2 = LD[2 * (qoff + myq)];
    dd = LD[2 * (qoff + myq) + 1];
  }
#pragma unroll
  for (int ks = 0; ks < kNKS; ++ks) {
    if (qvalid) {
      qv[ks] = *(const vec8*)(Q + (qoff + myq) * D + 16 * ks + 8 * hl);
      gv[ks] = *(const vec8*)(dO + (qoff + myq) * D + 16 * ks + 8 * hl);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) { qv[ks][e] = 0; gv[ks][e] = 0; }
    }
  }

  const int kv_end = CAUSAL ? min(S, q0 + BM) : S;
  const int n_tiles = (kv_end + BN - 1) / BN;
  // 32-key halves this wave computes; the last one holds the causal diagonal
  // or the end of the keys
  const int w_end = CAUSAL ? min(kv_end, qw0 + 32) : kv_end;
  const int w_halves = qw0 < S ? (w_end + 31) / 32 : 0;

  // HBM -> LDS: load i of this wave covers the kRpk tile rows from
  // kRpk (kDma wave + i); rows at or past kv_end read as zero.
  const uint32_t kv_bytes = (uint32_t)kv_end * kRowB;
  uint32_t dma_off[kDma];
#pragma unroll
  for (int i = 0; i < kDma; ++i) {
    dma_off[i] = Gm::dma_ofs(Gm::kRpk * (kDma * wave + i), lane);
  }
  auto issue = [&](int tt) CA_INLINE {
    unsigned char* dst = lds + (tt % kStages) * kStageB + wave * (kDma * 1024);
    const uint32_t toff = (uint32_t)tt * kTileB;
    const __amdgpu_buffer_rsrc_t k_rsrc = make_rsrc_at(Kp, toff, kv_bytes);
    const __amdgpu_buffer_rsrc_t v_rsrc = make_rsrc_at(Vp, toff, kv_bytes);
#pragma unroll
    for (int i = 0; i < kDma; ++i) {
      dma16_buf(k_rsrc, (CA_LDS void*)(dst + 1024 * i), dma_off[i]);
      dma16_buf(v_rsrc, (CA_LDS void*)(dst + kTileB + 1024 * i), dma_off[i]);
    }
  };
  const uint32_t lds0 = lds_off(lds);
  const uint32_t rofs = Gm::row_ofs(rho32(l32), hl);
  const TrOfs tofs = Gm::tr_ofs(lane);

  f32x16 acc[kNOB];  // dQ^T: rows d = 32 ob + .., column = this lane's query
#pragma unroll
  for (int i = 0; i < kNOB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

  // One half of 32 keys (k0 = first key) at LDS byte `hb` (K rows; V rows at
  // hb + kTileB).
  // (only the softmax step differs between masked and unmasked halves)
  auto half = [&](uint32_t hb, int k0, bool mask) CA_INLINE {
    // S^T = K Q^T, dP^T = V dO^T: register r of half hl <-> key
    // k0 + 16 (r/8) + 8 hl + r%8, column = this lane's query
    f32x16 s, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) { s[r] = 0.f; dp[r] = 0.f; }
    const uint32_t ka = hb + rofs, va = ka + kTileB;
    u32x4 kr[2], vr[2];
    kr[0] = lds_read_b128<0>(ka);
    vr[0] = lds_read_b128<0>(va);
#pragma unroll
    for (int ks = 0; ks < kNKS; ++ks) {
      const int cb = ks & 1;
      if (ks < kNKS - 1) {
        kr[cb ^ 1] = lds_read_b128<0>(ka ^ (32 * (ks + 1)));
        vr[cb ^ 1] = lds_read_b128<0>(va ^ (32 * (ks + 1)));
        wait_lgkm<2>();
      } else {
        wait_lgkm<0>();
      }
      after_wait(kr[cb]);
      after_wait(vr[cb]);
      s = Tr::mfma32(__builtin_bit_cast(vec8, kr[cb]), qv[ks], s);
      dp = Tr::mfma32(__builtin_bit_cast(vec8, vr[cb]), gv[ks], dp);
    }
    // dS^T / scale = P (dP - D) as the B operand of dQ^T += K^T dS^T
    vec8 pb[2];
    auto softmax = [&](auto mask_tag) CA_INLINE {
    constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float ds[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int r = 8 * kk + 2 * j + e;
          float p = fast_exp2(__builtin_fmaf(s[r], c2, -lse2));
          if (MASK) {
            const int key = k0 + 16 * kk + 8 * hl + 2 * j + e;
            if (key >= S || (CAUSAL && key > myq)) p = 0.f;
          }
          ds[e] = p * (dp[r] - dd);
        }
        const vec2 pk = Tr::pack2(ds[0], ds[1]);
        pb[kk][2 * j] = pk[0];
        pb[kk][2 * j + 1] = pk[1];
      }
    }
    };
    if (mask) softmax(std::true_type{});
    else softmax(std::false_type{});
    // dQ^T[d x q] += K^T[d x keys] dS^T[keys x q]
#pragma unroll
    for (int ob = 0; ob < kNOB; ++ob) {
      const vec8 a0 = Gm::template tr_operand<Tr, 0>(hb, tofs, ob);
      const vec8 a1 = Gm::template tr_operand<Tr, 1>(hb, tofs, ob);
      wait_lgkm<0>();
      vec8 x0 = a0, x1 = a1;
      after_wait(x0);
      after_wait(x1);
      acc[ob] = Tr::mfma32(x0, pb[0], acc[ob]);
      acc[ob] = Tr::mfma32(x1, pb[1], acc[ob]);
    }
  };

#pragma unroll
  for (int tt = 0; tt < kDist; ++tt) issue(tt);
  for (int t = 0; t < n_tiles; ++t) {
    wait_vmcnt<2 * kDma * (kDist - 1)>();  // this wave's loads of tile t landed
    __builtin_amdgcn_s_barrier();          // ... and every wave's; slot of t-1 is free
    issue(t + kDist);
    const uint32_t sb = lds0 + (uint32_t)((t % kStages) * kStageB);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int j = 2 * t + hh;
      if (j < w_halves) {
        half(sb + hh * 32 * kRowB, 32 * j, CAUSAL ? (j == w_halves - 1) : (32 * j + 32 > S));
      }
    }
  }
  wait_vmcnt<0>();  // no load may still target this workgroup's LDS when it exits
  store_rowsT_lds<Tr, kNOB, 128>(dQ + qoff * D, qw0, S, acc, scale,
                                 lds_off(qstg) + (uint32_t)(wave * 32 * 128), lane);
}

template <typename Tr, int D, bool CAUSAL>
__global__ __launch_bounds__(64 * bwdma::kNW) void bwd_dq_dma_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, const uint16_t* __restrict__ dO,
    const float* __restrict__ LD, uint16_t* __restrict__ dQ, int S, int Hq, int Hkv, float scale,
    int n_qt, int n_bh, int n_work, int paired) {
  const QTileWork wk =
      prefill_work(xcd_remap(__builtin_amdgcn_workgroup_id_x(), n_work), n_qt, n_bh, paired);
  const int n_pass = wk.qt1 < 0 ? 1 : 2;
#pragma clang loop unroll(disable)
  for (int pass = 0; pass < n_pass; ++pass) {
    if (pass) __builtin_amdgcn_s_barrier();  // every wave is done reading the ring
    bwd_dq_dma_tile<Tr, D, CAUSAL>(Q, K, V, dO, LD, dQ, S, Hq, Hkv, scale, pass ? wk.bh1 : wk.bh0,
                               pass ? wk.qt1 : wk.qt0);
  }
}

// dK, dV of key tile kt (256 keys) of kv head bhk: every q head of the kv head,
// queries in tiles of 32 (from the tile holding the first key when causal).
// K^T stays in registers; each wave keeps its own 32 V rows in LDS (the V^T B
// operand of dP); Q, dO and the (LSE log2 e, D) pairs stream through the ring.
template <typename Tr, int D, bool CAUSAL>
__device__ CA_INLINE void bwd_dkv_dma_tile(const uint16_t* __restrict__ Q,
                                          const uint16_t* __restrict__ K,
                                          const uint16_t* __restrict__ V,
                                          const uint16_t* __restrict__ dO,
                                          const float* __restrict__ LD, uint16_t* __restrict__ dK,
                                          uint16_t* __restrict__ dV, int S, int Hq, int Hkv,
                                          float scale, int bhk, int kt) {
  using namespace bwdma;
  using Gm = Geom<D>;
  using vec8 = typename Tr::vec8;
  using vec2 = typename Tr::vec2;
  constexpr int kRowB = Gm::kRowB, kNKS = Gm::kNKS, kNOB = Gm::kNOB;
  constexpr int BK = 32 * kNW;                  // keys per workgroup
  constexpr int BQ = 32;                        // queries per ring tile
  constexpr int kTileB = BQ * kRowB;            // 8 KB (D = 128), 4 KB (D = 64)
  constexpr int kStageB = 2 * kTileB + 1024;    // Q tile, dO tile, pairs
  constexpr int kVB = 32 * kRowB;               // V rows of one wave
  // D = 128: every wave loads 1 KB of the Q tile and 1 KB of the dO tile;
  // D = 64: waves 0..3 load the Q tile, waves 4..7 the dO tile
  constexpr bool kSplit = kTileB < 1024 * kNW;
  static_assert(kTileB == 1024 * kNW || 2 * kTileB == 1024 * kNW, "whole 1-KB loads per wave");
  constexpr int kLoads = kSplit ? 1 : 2;        // ring loads per wave per tile (+1: pairs, wave 0)
  __shared__ __attribute__((aligned(1024))) unsigned char lds[kNW * kVB + kStages * kStageB];

  const int b = bhk / Hkv, hk = bhk % Hkv;
  const int G = Hq / Hkv;
  const int K0 = kt * BK;
  const size_t kvoff = (size_t)(b * Hkv + hk) * S;
  // The lane index is recomputed per call (lane_here): otherwise the
  // compiler hoists the lane-derived load offsets of both passes out of the
  // kernel's pass loop and keeps them live through the tile loop, which at
  // 256 VGPRs spills them (measured: 13-14 spilled registers at D = 128).
  const int lane = lane_here();
  const int wave = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_workitem_id_x() >> 6);
  const int l32 = lane & 31, hl = lane >> 5;
  const int kw0 = K0 + 32 * wave;
  const int mykey = kw0 + l32;
  const bool kvalid = mykey < S;
  const float c2 = scale * kLog2e;

  // this wave's V rows -> LDS (rows past S read as zero)
  unsigned char* vw = lds + wave * kVB;
  {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(V + kvoff * D, (uint32_t)S * kRowB);
#pragma unroll
    for (int i = 0; i < kVB / 1024; ++i)
      dma16_buf(rs, (CA_LDS void*)(vw + 1024 * i),
                (uint32_t)kw0 * kRowB + Gm::dma_ofs(Gm::kRpk * i, lane));
  }
  vec8 kv[kNKS];  // K^T as the B operand of S = Q K^T (column = this lane's key)
#pragma unroll
  for (int ks = 0; ks < kNKS; ++ks) {
    if (kvalid) {
      kv[ks] = *(const vec8*)(K + (kvoff + mykey) * D + 16 * ks + 8 * hl);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) kv[ks][e] = 0;
    }
  }

  const int t_begin = CAUSAL ? K0 / BQ : 0;
  const int nt = max(0, (S + BQ - 1) / BQ - t_begin);  // query tiles per q head
  const int n_it = G * nt;
  // ring load of tile it: 1-KB loads of Q and dO (tile rows from kRpk wsub),
  // the 64 floats of pairs by wave 0
  const int wsub = kSplit ? (wave & (kNW / 2 - 1)) : wave;
  const uint32_t dma_off = Gm::dma_ofs(Gm::kRpk * wsub, lane);
  auto issue = [&](int it) CA_INLINE {
    unsigned char* st = lds + kNW * kVB + (it % kStages) * kStageB;
    // past the walk (slots the loop never reads): offsets past the slice, zeros
    const bool past = it >= n_it;
    const int itc = past ? 0 : it;
    const int h = hk * G + itc / max(nt, 1);
    const int q0 = past ? S : (t_begin + itc % max(nt, 1)) * BQ;
    const size_t ho = (size_t)(b * Hq + h) * S;
    const uint32_t qoff = (uint32_t)q0 * kRowB, sz = (uint32_t)S * kRowB;
    if (!kSplit || wave < kNW / 2)
      dma16_buf(make_rsrc_at(Q + ho * D, qoff, sz), (CA_LDS void*)(st + 1024 * wsub), dma_off);
    if (!kSplit || wave >= kNW / 2)
      dma16_buf(make_rsrc_at(dO + ho * D, qoff, sz), (CA_LDS void*)(st + kTileB + 1024 * wsub),
                dma_off);
    if (wave == 0)
      dma4_buf(make_rsrc_at(LD + 2 * ho, (uint32_t)q0 * 8, (uint32_t)S * 8),
               (CA_LDS void*)(st + 2 * kTileB), 4 * lane);
  };
  const uint32_t lds0 = lds_off(lds);
  const uint32_t rofs = Gm::row_ofs(rho32(l32), hl);  // Q / dO rows (A operands)
  const uint32_t vofs = lds0 + wave * kVB + Gm::row_ofs(l32, hl);  // V rows (B operand)
  const TrOfs tofs = Gm::tr_ofs(lane);

  f32x16 dk[kNOB], dv[kNOB];  // dK^T, dV^T: rows d = 32 ob + .., column = this lane's key
#pragma unroll
  for (int i = 0; i < kNOB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) { dk[i][r] = 0.f; dv[i][r] = 0.f; }

  // One query tile at LDS byte `sb`; only the softmax step differs between
  // masked and unmasked tiles (a branch around the whole tile doubles the
  // registers the compiler keeps live).
  auto tile = [&](uint32_t sb, int q0, bool mask) CA_INLINE {
    // S = Q K^T, dP = dO V^T: register r of half hl <-> query
    // q0 + 16 (r/8) + 8 hl + r%8, column = this lane's key
    f32x16 s, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) { s[r] = 0.f; dp[r] = 0.f; }
    const uint32_t qa = sb + rofs, ga = qa + kTileB;
    u32x4 qr[2], gr[2], vr[2];
    qr[0] = lds_read_b128<0>(qa);
    gr[0] = lds_read_b128<0>(ga);
    vr[0] = lds_read_b128<0>(vofs);
#pragma unroll
    for (int ks = 0; ks < kNKS; ++ks) {
      const int cb = ks & 1;
      if (ks < kNKS - 1) {
        qr[cb ^ 1] = lds_read_b128<0>(qa ^ (32 * (ks + 1)));
        gr[cb ^ 1] = lds_read_b128<0>(ga ^ (32 * (ks + 1)));
        vr[cb ^ 1] = lds_read_b128<0>(vofs ^ (32 * (ks + 1)));
        wait_lgkm<3>();
      } else {
        wait_lgkm<0>();
      }
      after_wait(qr[cb]);
      after_wait(gr[cb]);
      after_wait(vr[cb]);
      s = Tr::mfma32(__builtin_bit_cast(vec8, qr[cb]), kv[ks], s);
      dp = Tr::mfma32(__builtin_bit_cast(vec8, gr[cb]), __builtin_bit_cast(vec8, vr[cb]), dp);
    }
    // P and dS / scale = P (dP - D) as B operands, k-step kk = 16 queries
    vec8 pp[2], pd[2];
    auto softmax = [&](auto mask_tag) CA_INLINE {
    constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      // pairs of queries 16 kk + 8 hl + 0..7
      const uint32_t la = sb + 2 * kTileB + 8 * (16 * kk + 8 * hl);
      u32x4 w[4] = {lds_read_b128<0>(la), lds_read_b128<16>(la), lds_read_b128<32>(la),
                    lds_read_b128<48>(la)};
      wait_lgkm<0>();
#pragma unroll
      for (int i = 0; i < 4; ++i) after_wait(w[i]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float p[2], ds[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int r = 8 * kk + 2 * j + e;
          // element copies first: clang's __builtin_bit_cast of a vector
          // element at a nonzero index reads element 0
          const uint32_t lw = w[j][2 * e], dw = w[j][2 * e + 1];
          const float l2 = __builtin_bit_cast(float, lw);
          const float dd = __builtin_bit_cast(float, dw);
          p[e] = fast_exp2(__builtin_fmaf(s[r], c2, -l2));
          if (MASK) {
            const int query = q0 + 16 * kk + 8 * hl + 2 * j + e;
            if (query >= S || (CAUSAL && mykey > query)) p[e] = 0.f;
          }
          ds[e] = p[e] * (dp[r] - dd);
        }
        const vec2 a = Tr::pack2(p[0], p[1]);
        const vec2 c = Tr::pack2(ds[0], ds[1]);
        pp[kk][2 * j] = a[0];
        pp[kk][2 * j + 1] = a[1];
        pd[kk][2 * j] = c[0];
        pd[kk][2 * j + 1] = c[1];
      }
    }
    };
    if (mask) softmax(std::true_type{});
    else softmax(std::false_type{});
    // dV^T[d x keys] += dO^T P and dK^T[d x keys] += Q^T dS
#pragma unroll
    for (int ob = 0; ob < kNOB; ++ob) {
      const vec8 g0 = Gm::template tr_operand<Tr, 0>(sb + kTileB, tofs, ob);
      const vec8 g1 = Gm::template tr_operand<Tr, 1>(sb + kTileB, tofs, ob);
      const vec8 x0 = Gm::template tr_operand<Tr, 0>(sb, tofs, ob);
      const vec8 x1 = Gm::template tr_operand<Tr, 1>(sb, tofs, ob);
      wait_lgkm<0>();
      vec8 a0 = g0, a1 = g1, b0 = x0, b1 = x1;
      after_wait(a0);
      after_wait(a1);
      after_wait(b0);
      after_wait(b1);
      dv[ob] = Tr::mfma32(a0, pp[0], dv[ob]);
      dk[ob] = Tr::mfma32(b0, pd[0], dk[ob]);
      dv[ob] = Tr::mfma32(a1, pp[1], dv[ob]);
      dk[ob] = Tr::mfma32(b1, pd[1], dk[ob]);
    }
  };

#pragma unroll
  for (int i = 0; i < kDist; ++i) issue(i);
  for (int it = 0; it < n_it; ++it) {
    // this wave's loads of tile it (and its V rows, issued first) landed
    if (wave == 0) wait_vmcnt<(kLoads + 1) * (kDist - 1)>();
    else wait_vmcnt<kLoads * (kDist - 1)>();
    __builtin_amdgcn_s_barrier();  // ... and every wave's; slot of it-1 is free
    issue(it + kDist);
    const int q0 = (t_begin + it % nt) * BQ;
    if (kw0 < S && (!CAUSAL || q0 >= kw0)) {  // causal: queries before every key of the wave
      const uint32_t sb = lds0 + kNW * kVB + (uint32_t)((it % kStages) * kStageB);
      tile(sb, q0, (CAUSAL && q0 == kw0) || q0 + BQ > S);
    }
  }
  wait_vmcnt<0>();  // no load may still target this workgroup's LDS when it exits
  // the wave's V rows are no longer read: their LDS block stages dK, then dV
  store_rowsT_lds<Tr, kNOB, kRowB>(dK + kvoff * D, kw0, S, dk, scale, lds_off(vw), lane_here());
  store_rowsT_lds<Tr, kNOB, kRowB>(dV + kvoff * D, kw0, S, dv, 1.f, lds_off(vw), lane_here());
}

template <typename Tr, int D, bool CAUSAL>
__global__ __launch_bounds__(64 * bwdma::kNW) void bwd_dkv_dma_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, const uint16_t* __restrict__ dO,
    const float* __restrict__ LD, uint16_t* __restrict__ dK, uint16_t* __restrict__ dV, int S,
    int Hq, int Hkv, float scale, int n_kt, int n_bh, int n_work, int paired) {
  // key tile kt walks n_kt - kt query stretches: kt = n_kt - 1 - qt gives the
  // longest walks first (unpaired) and pairs of equal total length (paired)
  const QTileWork wk =
      prefill_work(xcd_remap(__builtin_amdgcn_workgroup_id_x(), n_work), n_kt, n_bh, paired);
  const int n_pass = wk.qt1 < 0 ? 1 : 2;
#pragma clang loop unroll(disable)
  for (int pass = 0; pass < n_pass; ++pass) {
    if (pass) __builtin_amdgcn_s_barrier();  // every wave is done reading the ring and V
    bwd_dkv_dma_tile<Tr, D, CAUSAL>(Q, K, V, dO, LD, dK, dV, S, Hq, Hkv, scale,
                                pass ? wk.bh1 : wk.bh0, n_kt - 1 - (pass ? wk.qt1 : wk.qt0));
  }
}

template <typename Tr, int D, bool CAUSAL>
hipError_t launch_bwd_t(const void* q, const void* k, const void* v, const void* o,
                        const void* dout, const float* lse, void* dq, void* dk, void* dv, int B,
                        int Hq, int Hkv, int S, float scale, float* ws, hipStream_t stream) {
  const long long rows = (long long)B * Hq * S;
  const long long threads = rows * (D / 8);
  const long long g0 = (threads + 255) / 256;
  if (g0 > 0x7fffffffLL) return hipErrorInvalidValue;
  // 256 keys (dK, dV) / 256 queries (dQ) per workgroup, one workgroup per CU
  constexpr int BT = 32 * bwdma::kNW;
  const int n_t = (S + BT - 1) / BT;
  int pk = 0, pq = 0;
  const long long gk = prefill_grid(B, Hkv, n_t, CAUSAL, 1, &pk);
  const long long gq = prefill_grid(B, Hq, n_t, CAUSAL, 1, &pq);
  if (gk > 0x7fffffffLL || gq > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((bwd_rowdot_kernel<Tr, D>), dim3((unsigned)g0), dim3(256), 0, stream,
                     (const uint16_t*)o, (const uint16_t*)dout, lse, ws, rows);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((bwd_dkv_dma_kernel<Tr, D, CAUSAL>), dim3((unsigned)gk), dim3(64 * bwdma::kNW),
                     0, stream, (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,
                     (const uint16_t*)dout, ws, (uint16_t*)dk, (uint16_t*)dv, S, Hq, Hkv, scale,
                     n_t, B * Hkv, (int)gk, pk);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((bwd_dq_dma_kernel<Tr, D, CAUSAL>), dim3((unsigned)gq), dim3(64 * bwdma::kNW),
                     0, stream, (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,
                     (const uint16_t*)dout, ws, (uint16_t*)dq, S, Hq, Hkv, scale, n_t, B * Hq,
                     (int)gq, pq);
  return hipGetLastError();
}

}  // namespace

size_t bwd_workspace_bytes(int B, int Hq, int S) { return (size_t)B * Hq * S * 2 * sizeof(float); }

hipError_t launch_flash_bwd(int dtype, const void* q, const void* k, const void* v,
                            const void* o, const void* dout, const float* lse, void* dq, void* dk,
                            void* dv, int B, int Hq, int Hkv, int S, int D, float scale,
                            bool causal, void* ws, hipStream_t stream) {
  if ((long long)B * Hq * S == 0) return hipSuccess;
  if (dtype == kDtypeF32)
    return launch_flash_bwd_f32((const float*)q, (const float*)k, (const float*)v, (const float*)o,
                                (const float*)dout, lse, (float*)dq, (float*)dk, (float*)dv, B,
                                Hq, Hkv, S, D, scale, causal, ws, stream);
  float* w = (float*)ws;
#define CA_BWD_CASE(TR, DD)                                                                   \
  if (D == DD)                                                                                \
    return causal ? launch_bwd_t<TR, DD, true>(q, k, v, o, dout, lse, dq, dk, dv, B, Hq, Hkv, \
                                               S, scale, w, stream)                           \
                  : launch_bwd_t<TR, DD, false>(q, k, v, o, dout, lse, dq, dk, dv, B, Hq,     \
                                                Hkv, S, scale, w, stream);
  if (dtype == kDtypeBF16) {
    CA_BWD_CASE(BF16, 64)
    CA_BWD_CASE(BF16, 128)
  } else if (dtype == kDtypeF16) {
    CA_BWD_CASE(F16, 64)
    CA_BWD_CASE(F16, 128)
  }
#undef CA_BWD_CASE
  return hipErrorInvalidValue;
}

}  // namespace ca
