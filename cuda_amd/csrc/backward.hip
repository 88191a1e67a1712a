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
//   bwd_rowdot_kernel  D = rowsum(dO * O) into a [B, Hq, S] fp32 workspace;
//   bwd_dq_kernel      query-outer: 4 waves x 32 queries of one (b, h); key
//                      tiles of 64 staged in LDS; per tile S^T = K Q^T,
//                      dP^T = V dO^T, dS^T, dQ^T += K^T dS^T;
//   bwd_dkv_kernel     key-outer: 4 waves x 32 keys of one (b, kv head); query
//                      tiles of 64 (Q, dO, LSE, D) staged in LDS, for every q
//                      head of the kv head; per tile S = Q K^T, dP = dO V^T,
//                      dS, dV^T += dO^T P, dK^T += Q^T dS.
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

#ifndef CA_BWD_DMA
#define CA_BWD_DMA 1
#endif
constexpr bool kBwdDma = CA_BWD_DMA != 0;  // head dim 128: the buffer-load kernels below
#ifndef CA_BWD_PRIO
#define CA_BWD_PRIO 0
#endif
constexpr int kBwdWaves = 4;    // waves per workgroup (32 rows each)
constexpr int kBwdTile = 64;    // keys (dq kernel) or queries (dkv kernel) per LDS tile

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

// Store the transposed accumulators acc[ob] (rows d = 32 ob + 8 a + 4 h + 0..3,
// column = this lane's row index l32) as row `row` of a [.., D] 16-bit tensor.
template <typename Tr, int NOB>
__device__ __forceinline__ void store_rowT(uint16_t* dst_row, const f32x16 (&acc)[NOB], int hl,
                                           float mul = 1.f) {
  using vec4 = typename Tr::vec4;
  using vec2 = typename Tr::vec2;
#pragma unroll
  for (int ob = 0; ob < NOB; ++ob) {
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int d = 32 * ob + 8 * a + 4 * hl;
      const vec2 lo = Tr::pack2(acc[ob][4 * a] * mul, acc[ob][4 * a + 1] * mul);
      const vec2 hi = Tr::pack2(acc[ob][4 * a + 2] * mul, acc[ob][4 * a + 3] * mul);
      vec4 w;
      w[0] = lo[0]; w[1] = lo[1]; w[2] = hi[0]; w[3] = hi[1];
      *(vec4*)(dst_row + d) = w;
    }
  }
}

// ---------------------------------------------------------------------------
// dQ: one workgroup = 128 queries of one (b, h); the key walk of the forward.
// ---------------------------------------------------------------------------
template <typename Tr, int D, bool CAUSAL>
__global__ __launch_bounds__(kBwdWaves * 64) void bwd_dq_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, const uint16_t* __restrict__ dO,
    const float* __restrict__ LD, uint16_t* __restrict__ dQ, int S, int Hq, int Hkv, float scale,
    int n_qt, int n_work) {
  using vec8 = typename Tr::vec8;
  using vec4 = typename Tr::vec4;
  using vec2 = typename Tr::vec2;
  constexpr int BM = 32 * kBwdWaves;
  constexpr int BN = kBwdTile;
  constexpr int KS = D + 8;   // row stride (elements): permuted-row b128 reads hit distinct banks
  constexpr int NKS = D / 16;
  constexpr int NOB = D / 32;
  constexpr int CHUNKS = D / 8;
  constexpr int ROWS_PER_PASS = kBwdWaves * 64 / CHUNKS;
  constexpr int PASSES = BN / ROWS_PER_PASS;
  static_assert(PASSES * ROWS_PER_PASS == BN, "tile staging must cover the tile");

  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][BN * KS];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][BN * KS];

  const int work = xcd_remap(blockIdx.x, n_work);
  const int bh = work / n_qt;
  const int qt = n_qt - 1 - (work % n_qt);  // longest causal walks first
  const int b = bh / Hq, h = bh % Hq;
  const int hk = h / (Hq / Hkv);
  const int q0 = qt * BM;
  const size_t qoff = (size_t)(b * Hq + h) * S;
  const uint16_t* Qp = Q + qoff * D;
  const uint16_t* dOp = dO + qoff * D;
  const uint16_t* Kp = K + (size_t)(b * Hkv + hk) * S * D;
  const uint16_t* Vp = V + (size_t)(b * Hkv + hk) * S * D;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, hl = lane >> 5;
  const int qw0 = q0 + 32 * wave;
  const int myq = qw0 + l32;
  const bool qvalid = myq < S;
  const float c2 = scale * kLog2e;
  // P = 2^(s * c2 - lse2); a query past S gets lse2 = +inf, so P = 0
  const float lse2 = qvalid ? LD[2 * (qoff + myq)] : -kNegInf;
  const float dd = qvalid ? LD[2 * (qoff + myq) + 1] : 0.f;

  vec8 qv[NKS], gv[NKS];  // Q and dO as B operands (column = this lane's query)
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    if (qvalid) {
      qv[ks] = *(const vec8*)(Qp + (size_t)myq * D + 16 * ks + 8 * hl);
      gv[ks] = *(const vec8*)(dOp + (size_t)myq * D + 16 * ks + 8 * hl);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) { qv[ks][e] = 0; gv[ks][e] = 0; }
    }
  }

  const int kv_end = CAUSAL ? min(S, q0 + BM) : S;
  const int n_tiles = (kv_end + BN - 1) / BN;
  const int st_row = tid / CHUNKS, st_col = (tid % CHUNKS) * 8;
  u32x4 kreg[PASSES], vreg[PASSES];
  auto gload = [&](int t) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int row = t * BN + st_row + p * ROWS_PER_PASS;
      if (row < S) {
        kreg[p] = *(const u32x4*)(Kp + (size_t)row * D + st_col);
        vreg[p] = *(const u32x4*)(Vp + (size_t)row * D + st_col);
      } else {
        kreg[p] = u32x4{0, 0, 0, 0};
        vreg[p] = u32x4{0, 0, 0, 0};
      }
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int r = st_row + p * ROWS_PER_PASS;
      *(u32x4*)(&Ks[buf][r * KS + st_col]) = kreg[p];
      *(u32x4*)(&Vs[buf][r * KS + st_col]) = vreg[p];
    }
  };

  f32x16 acc[NOB];  // dQ^T
#pragma unroll
  for (int i = 0; i < NOB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;

  const int krow = rho32(l32);
  const int g16 = lane >> 4, s16 = lane & 15;
  const int tr_row = 8 * (g16 >> 1) + (s16 >> 2);
  const int tr_col = 16 * (g16 & 1) + 4 * (s16 & 3);

  if (n_tiles > 0) gload(0);
  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    lstore(buf);
    __syncthreads();
    if (t + 1 < n_tiles) gload(t + 1);
    const int k0 = t * BN;
    if (CAUSAL && k0 > qw0 + 31) continue;  // tile entirely above this wave's rows
    const uint16_t* Kb = Ks[buf];
    const uint16_t* Vb = Vs[buf];

    // S^T = K Q^T and dP^T = V dO^T; register r of half hl <-> key
    // k0 + 32 mb + 16 (r/8) + 8 hl + r%8, column = this lane's query
    f32x16 s[2], dp[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) { s[mb][r] = 0.f; dp[mb][r] = 0.f; }
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const int off = (32 * mb + krow) * KS + 16 * ks + 8 * hl;
        s[mb] = Tr::mfma32(*(const vec8*)(Kb + off), qv[ks], s[mb]);
        dp[mb] = Tr::mfma32(*(const vec8*)(Vb + off), gv[ks], dp[mb]);
      }
    }
    const bool need_mask = CAUSAL ? (k0 + BN - 1 > qw0) : (k0 + BN > S);
    vec8 pb[4];  // dS^T as the B operand of dQ^T += K^T dS^T, k-step kk
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float ds[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int i = 8 * kk + 2 * j + e;  // register index over both blocks: mb = i / 16
          const int mb = i >> 4, r = i & 15;
          float p = fast_exp2(__builtin_fmaf(s[mb][r], c2, -lse2));
          if (need_mask) {
            const int key = k0 + 32 * mb + 16 * (r >> 3) + 8 * hl + (r & 7);
            if (key >= S || (CAUSAL && key > myq)) p = 0.f;
          }
          ds[e] = p * (dp[mb][r] - dd) * scale;
        }
        const vec2 pk = Tr::pack2(ds[0], ds[1]);
        pb[kk][2 * j] = pk[0];
        pb[kk][2 * j + 1] = pk[1];
      }
    }
    // dQ^T[d x q] += K^T[d x keys] dS^T[keys x q]
#pragma unroll
    for (int ob = 0; ob < NOB; ++ob) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const uint16_t* src = Kb + (16 * kk + tr_row) * KS + 32 * ob + tr_col;
        const vec4 lo = Tr::tr_read((const CA_LDS void*)src);
        const vec4 hi = Tr::tr_read((const CA_LDS void*)(src + 4 * KS));
        acc[ob] = Tr::mfma32(cat4<vec8, vec4>(lo, hi), pb[kk], acc[ob]);
      }
    }
  }
  if (qvalid) store_rowT<Tr, NOB>(dQ + (qoff + myq) * D, acc, hl);
}

// ---------------------------------------------------------------------------
// dK, dV: one workgroup = 128 keys of one (b, kv head); query tiles of every
// q head of the kv head.
// ---------------------------------------------------------------------------
template <typename Tr, int D, bool CAUSAL>
__global__ __launch_bounds__(kBwdWaves * 64) void bwd_dkv_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, const uint16_t* __restrict__ dO,
    const float* __restrict__ LD, uint16_t* __restrict__ dK, uint16_t* __restrict__ dV, int S,
    int Hq, int Hkv, float scale, int n_kt, int n_work) {
  using vec8 = typename Tr::vec8;
  using vec4 = typename Tr::vec4;
  using vec2 = typename Tr::vec2;
  constexpr int BK = 32 * kBwdWaves;  // keys per workgroup
  constexpr int BQ = kBwdTile;        // queries per LDS tile
  constexpr int KS = D + 8;
  constexpr int NKS = D / 16;
  constexpr int NOB = D / 32;
  constexpr int CHUNKS = D / 8;
  constexpr int ROWS_PER_PASS = kBwdWaves * 64 / CHUNKS;
  constexpr int PASSES = BQ / ROWS_PER_PASS;
  static_assert(PASSES * ROWS_PER_PASS == BQ, "tile staging must cover the tile");

  __shared__ __attribute__((aligned(16))) uint16_t Qs[2][BQ * KS];
  __shared__ __attribute__((aligned(16))) uint16_t Gs[2][BQ * KS];  // dO
  __shared__ __attribute__((aligned(16))) float Ls[2][BQ];          // LSE * log2(e)
  __shared__ __attribute__((aligned(16))) float Ds[2][BQ];          // D

  const int work = xcd_remap(blockIdx.x, n_work);
  const int bhk = work / n_kt;
  const int kt = work % n_kt;  // causal: the first key tiles have the longest query walks
  const int b = bhk / Hkv, hk = bhk % Hkv;
  const int G = Hq / Hkv;
  const int K0 = kt * BK;
  const uint16_t* Kp = K + (size_t)(b * Hkv + hk) * S * D;
  const uint16_t* Vp = V + (size_t)(b * Hkv + hk) * S * D;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, hl = lane >> 5;
  const int kw0 = K0 + 32 * wave;
  const int mykey = kw0 + l32;
  const bool kvalid = mykey < S;
  const float c2 = scale * kLog2e;

  vec8 kv[NKS], vv[NKS];  // K^T and V^T as B operands (column = this lane's key)
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    if (kvalid) {
      kv[ks] = *(const vec8*)(Kp + (size_t)mykey * D + 16 * ks + 8 * hl);
      vv[ks] = *(const vec8*)(Vp + (size_t)mykey * D + 16 * ks + 8 * hl);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) { kv[ks][e] = 0; vv[ks][e] = 0; }
    }
  }

  // query tiles: causal walks start at the tile holding the first key
  const int t_begin = CAUSAL ? K0 / BQ : 0;
  const int t_end = (S + BQ - 1) / BQ;
  const int nt = max(0, t_end - t_begin);
  const int n_it = G * nt;

  const int st_row = tid / CHUNKS, st_col = (tid % CHUNKS) * 8;
  u32x4 qreg[PASSES], greg[PASSES];
  float lreg = 0.f, dreg = 0.f;
  auto gload = [&](int it) {
    const int h = hk * G + it / nt;
    const int q0 = (t_begin + it % nt) * BQ;
    const size_t qoff = (size_t)(b * Hq + h) * S;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int row = q0 + st_row + p * ROWS_PER_PASS;
      if (row < S) {
        qreg[p] = *(const u32x4*)(Q + (qoff + row) * D + st_col);
        greg[p] = *(const u32x4*)(dO + (qoff + row) * D + st_col);
      } else {
        qreg[p] = u32x4{0, 0, 0, 0};
        greg[p] = u32x4{0, 0, 0, 0};
      }
    }
    if (tid < BQ) {
      const int row = q0 + tid;
      lreg = row < S ? LD[2 * (qoff + row)] : -kNegInf;  // past S: P = 0
      dreg = row < S ? LD[2 * (qoff + row) + 1] : 0.f;
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int r = st_row + p * ROWS_PER_PASS;
      *(u32x4*)(&Qs[buf][r * KS + st_col]) = qreg[p];
      *(u32x4*)(&Gs[buf][r * KS + st_col]) = greg[p];
    }
    if (tid < BQ) {
      Ls[buf][tid] = lreg;
      Ds[buf][tid] = dreg;
    }
  };

  f32x16 dk[NOB], dv[NOB];  // dK^T, dV^T
#pragma unroll
  for (int i = 0; i < NOB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) { dk[i][r] = 0.f; dv[i][r] = 0.f; }

  const int qrow = rho32(l32);
  const int g16 = lane >> 4, s16 = lane & 15;
  const int tr_row = 8 * (g16 >> 1) + (s16 >> 2);
  const int tr_col = 16 * (g16 & 1) + 4 * (s16 & 3);

  if (n_it > 0) gload(0);
  for (int it = 0; it < n_it; ++it) {
    const int buf = it & 1;
    lstore(buf);
    __syncthreads();
    if (it + 1 < n_it) gload(it + 1);
    const int q0 = (t_begin + it % nt) * BQ;
    const uint16_t* Qb = Qs[buf];
    const uint16_t* Gb = Gs[buf];
#pragma unroll
    for (int qb = 0; qb < BQ / 32; ++qb) {
      const int qs = q0 + 32 * qb;  // first query of the 32-query block
      if (CAUSAL && qs + 31 < kw0) continue;  // every query before every key of the wave
      // S = Q K^T, dP = dO V^T; register r of half hl <-> query
      // qs + 16 (r/8) + 8 hl + r%8, column = this lane's key
      f32x16 s, dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) { s[r] = 0.f; dp[r] = 0.f; }
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int off = (32 * qb + qrow) * KS + 16 * ks + 8 * hl;
        s = Tr::mfma32(*(const vec8*)(Qb + off), kv[ks], s);
        dp = Tr::mfma32(*(const vec8*)(Gb + off), vv[ks], dp);
      }
      const bool need_mask = !kvalid || (CAUSAL && qs < kw0 + 31);
      vec8 pp[2], pd[2];  // P and dS as B operands, k-step kk = 16 queries
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int qi = 32 * qb + 16 * kk + 8 * hl;  // tile row of register 8 kk
        float lv[8], dv8[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) { lv[j] = Ls[buf][qi + j]; dv8[j] = Ds[buf][qi + j]; }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float p[2], ds[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int r = 8 * kk + 2 * j + e;
            p[e] = fast_exp2(__builtin_fmaf(s[r], c2, -lv[2 * j + e]));
            if (need_mask) {
              const int query = q0 + qi + 2 * j + e;
              if (!kvalid || (CAUSAL && mykey > query)) p[e] = 0.f;
            }
            ds[e] = p[e] * (dp[r] - dv8[2 * j + e]) * scale;
          }
          const vec2 a = Tr::pack2(p[0], p[1]);
          const vec2 c = Tr::pack2(ds[0], ds[1]);
          pp[kk][2 * j] = a[0];
          pp[kk][2 * j + 1] = a[1];
          pd[kk][2 * j] = c[0];
          pd[kk][2 * j + 1] = c[1];
        }
      }
      // dV^T[d x keys] += dO^T P and dK^T[d x keys] += Q^T dS
#pragma unroll
      for (int ob = 0; ob < NOB; ++ob) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const int off = (32 * qb + 16 * kk + tr_row) * KS + 32 * ob + tr_col;
          const vec4 glo = Tr::tr_read((const CA_LDS void*)(Gb + off));
          const vec4 ghi = Tr::tr_read((const CA_LDS void*)(Gb + off + 4 * KS));
          dv[ob] = Tr::mfma32(cat4<vec8, vec4>(glo, ghi), pp[kk], dv[ob]);
          const vec4 qlo = Tr::tr_read((const CA_LDS void*)(Qb + off));
          const vec4 qhi = Tr::tr_read((const CA_LDS void*)(Qb + off + 4 * KS));
          dk[ob] = Tr::mfma32(cat4<vec8, vec4>(qlo, qhi), pd[kk], dk[ob]);
        }
      }
    }
  }
  if (kvalid) {
    const size_t koff = ((size_t)(b * Hkv + hk) * S + mykey) * D;
    store_rowT<Tr, NOB>(dK + koff, dk, hl);
    store_rowT<Tr, NOB>(dV + koff, dv, hl);
  }
}

// ---------------------------------------------------------------------------
// Head dim 128: HBM -> LDS buffer loads, 8 waves (two per SIMD) per workgroup.
//
// Tiles are rows of 256 bytes stored unpadded with the 16-byte chunk c of row
// r at position c ^ swz(r), swz(r) = 4 (r % 4) + (r / 4) % 4 (the layout of
// the forward kernel), which keeps both read patterns bank-conflict free:
// row reads (ds_read_b128, one chunk of 16 consecutive rows per 16 lanes; the
// A operand of S^T / S and dP^T / dP, and the V^T B operand of dP) and
// transposed reads (ds_read_b64_tr_b16, 4 chunks of 4 consecutive rows per 32
// lanes; the K^T, Q^T and dO^T A operands). 1/scale is folded out of dS and
// applied once when dQ and dK are stored.
// ---------------------------------------------------------------------------
namespace bw128 {
constexpr int kD = 128;
constexpr int kRowB = kD * 2;  // bytes per row
constexpr int kNW = 8;         // waves per workgroup
constexpr int kStages = 4;     // ring tiles
constexpr int kDist = kStages - 1;
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
// Row-read byte offset: row `row`, logical chunk hl (XOR 32 * ks for chunk 2 ks + hl).
__device__ __forceinline__ uint32_t row_ofs(int row, int hl) {
  const int f = swz(row);
  return row * kRowB + 32 * (f >> 1) + 16 * (hl ^ (f & 1));
}
// Transposed-read byte offsets of a lane (rows 8 (g16/2) + s16/4 and +4 of a
// 16-row k-step, dims 32 ob + ..: XOR 64 ob), as in the forward's V^T reads.
struct TrOfs {
  uint32_t a, b;
};
__device__ __forceinline__ TrOfs tr_ofs(int lane) {
  const int g16 = lane >> 4, s16 = lane & 15;
  const int row = 8 * (g16 >> 1) + (s16 >> 2);
  const int c0 = 2 * (g16 & 1) + ((s16 & 3) >> 1);
  const int f = swz(row);  // swz(row + 4) == f + 1
  TrOfs t;
  t.a = row * kRowB + 64 * (f >> 2) + 16 * (c0 ^ (f & 3)) + 8 * (s16 & 1);
  t.b = (row + 4) * kRowB + 64 * (f >> 2) + 16 * (c0 ^ ((f + 1) & 3)) + 8 * (s16 & 1);
  return t;
}
// A operand (32 dims x 16 rows) of k-step kk of a tile at `base`, dims block ob.
template <typename Tr, int KK>
__device__ __forceinline__ typename Tr::vec8 tr_operand(uint32_t base, TrOfs t, int ob) {
  const u32x2 lo = lds_read_tr16<4096 * KK>((base + t.a) ^ (64 * ob));
  const u32x2 hi = lds_read_tr16<4096 * KK>((base + t.b) ^ (64 * ob));
  const u32x4 w = {lo[0], lo[1], hi[0], hi[1]};
  return __builtin_bit_cast(typename Tr::vec8, w);
}
}  // namespace bw128

// dQ of query tile qt (256 rows) of head bh: the keys [0, kv_end) in tiles of
// 64, each computed as two halves of 32 keys.
template <typename Tr, bool CAUSAL>
__device__ CA_INLINE void bwd_dq128_tile(const uint16_t* __restrict__ Q,
                                         const uint16_t* __restrict__ K,
                                         const uint16_t* __restrict__ V,
                                         const uint16_t* __restrict__ dO,
                                         const float* __restrict__ LD, uint16_t* __restrict__ dQ,
                                         int S, int Hq, int Hkv, float scale, int bh, int qt) {
  using namespace bw128;
  using vec8 = typename Tr::vec8;
  using vec2 = typename Tr::vec2;
  constexpr int BM = 32 * kNW;
  constexpr int BN = 64;
  constexpr int kTileB = BN * kRowB;           // 16 KB
  constexpr int kStageB = 2 * kTileB;          // K tile, then V tile
  constexpr int kDma = kTileB / 1024 / kNW;    // 1-KB loads per wave per K (and V) tile
  __shared__ __attribute__((aligned(1024))) unsigned char lds[kStages * kStageB];

  const int b = bh / Hq, h = bh % Hq;
  const int hk = h / (Hq / Hkv);
  const int q0 = qt * BM;
  const size_t qoff = (size_t)(b * Hq + h) * S;
  const uint16_t* Kp = K + (size_t)(b * Hkv + hk) * S * kD;
  const uint16_t* Vp = V + (size_t)(b * Hkv + hk) * S * kD;
  const int lane = __builtin_amdgcn_workitem_id_x() & 63;
  const int wave = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_workitem_id_x() >> 6);
  const int l32 = lane & 31, hl = lane >> 5;
  const int qw0 = q0 + 32 * wave;
  const int myq = qw0 + l32;
  const bool qvalid = myq < S;
  const float c2 = scale * kLog2e;
  float lse2 = -kNegInf, dd = 0.f;  // a query past S: P = 0
  vec8 qv[8], gv[8];                // Q and dO as B operands (column = this lane's query)
  if (qvalid) {
    lse2 = LD[2 * (qoff + myq)];
    dd = LD[2 * (qoff + myq) + 1];
  }
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    if (qvalid) {
      qv[ks] = *(const vec8*)(Q + (qoff + myq) * kD + 16 * ks + 8 * hl);
      gv[ks] = *(const vec8*)(dO + (qoff + myq) * kD + 16 * ks + 8 * hl);
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

  // HBM -> LDS: load i of this wave covers tile rows 4 (kDma wave + i) + lane/16,
  // the lane fetching the chunk that belongs at position lane % 16; rows at or
  // past kv_end read as zero.
  const uint32_t kv_bytes = (uint32_t)kv_end * kRowB;
  uint32_t dma_off[kDma];
#pragma unroll
  for (int i = 0; i < kDma; ++i) {
    const int row = 4 * (kDma * wave + i) + (lane >> 4);
    dma_off[i] = row * kRowB + 16 * ((lane & 15) ^ swz(row));
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
  const uint32_t rofs = row_ofs(rho32(l32), hl);
  const TrOfs tofs = tr_ofs(lane);

  f32x16 acc[4];  // dQ^T: rows d = 32 ob + .., column = this lane's query
#pragma unroll
  for (int i = 0; i < 4; ++i)
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
    if (CA_BWD_PRIO) __builtin_amdgcn_s_setprio(1);
    u32x4 kr[2], vr[2];
    kr[0] = lds_read_b128<0>(ka);
    vr[0] = lds_read_b128<0>(va);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const int cb = ks & 1;
      if (ks < 7) {
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
    if (CA_BWD_PRIO) __builtin_amdgcn_s_setprio(0);
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
    if (CA_BWD_PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) {
      const vec8 a0 = tr_operand<Tr, 0>(hb, tofs, ob);
      const vec8 a1 = tr_operand<Tr, 1>(hb, tofs, ob);
      wait_lgkm<0>();
      vec8 x0 = a0, x1 = a1;
      after_wait(x0);
      after_wait(x1);
      acc[ob] = Tr::mfma32(x0, pb[0], acc[ob]);
      acc[ob] = Tr::mfma32(x1, pb[1], acc[ob]);
    }
    if (CA_BWD_PRIO) __builtin_amdgcn_s_setprio(0);
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
  if (qvalid) store_rowT<Tr, 4>(dQ + (qoff + myq) * kD, acc, hl, scale);
}

template <typename Tr, bool CAUSAL>
__global__ __launch_bounds__(64 * bw128::kNW) void bwd_dq128_kernel(
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
    bwd_dq128_tile<Tr, CAUSAL>(Q, K, V, dO, LD, dQ, S, Hq, Hkv, scale, pass ? wk.bh1 : wk.bh0,
                               pass ? wk.qt1 : wk.qt0);
  }
}

// dK, dV of key tile kt (256 keys) of kv head bhk: every q head of the kv head,
// queries in tiles of 32 (from the tile holding the first key when causal).
// K^T stays in registers; each wave keeps its own 32 V rows in LDS (the V^T B
// operand of dP); Q, dO and the (LSE log2 e, D) pairs stream through the ring.
template <typename Tr, bool CAUSAL>
__device__ CA_INLINE void bwd_dkv128_tile(const uint16_t* __restrict__ Q,
                                          const uint16_t* __restrict__ K,
                                          const uint16_t* __restrict__ V,
                                          const uint16_t* __restrict__ dO,
                                          const float* __restrict__ LD, uint16_t* __restrict__ dK,
                                          uint16_t* __restrict__ dV, int S, int Hq, int Hkv,
                                          float scale, int bhk, int kt) {
  using namespace bw128;
  using vec8 = typename Tr::vec8;
  using vec2 = typename Tr::vec2;
  constexpr int BK = 32 * kNW;                  // keys per workgroup
  constexpr int BQ = 32;                        // queries per ring tile
  constexpr int kTileB = BQ * kRowB;            // 8 KB: one 1-KB load per wave
  constexpr int kLdB = BQ * 8;                  // (LSE log2 e, D) pairs
  constexpr int kStageB = 2 * kTileB + 1024;    // Q tile, dO tile, pairs
  constexpr int kVB = 32 * kRowB;               // V rows of one wave
  static_assert(kTileB == 1024 * kNW, "one 1-KB load per wave per Q (and dO) tile");
  __shared__ __attribute__((aligned(1024))) unsigned char lds[kNW * kVB + kStages * kStageB];

  const int b = bhk / Hkv, hk = bhk % Hkv;
  const int G = Hq / Hkv;
  const int K0 = kt * BK;
  const size_t kvoff = (size_t)(b * Hkv + hk) * S;
  const int lane = __builtin_amdgcn_workitem_id_x() & 63;
  const int wave = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_workitem_id_x() >> 6);
  const int l32 = lane & 31, hl = lane >> 5;
  const int kw0 = K0 + 32 * wave;
  const int mykey = kw0 + l32;
  const bool kvalid = mykey < S;
  const float c2 = scale * kLog2e;

  // this wave's V rows -> LDS (rows past S read as zero)
  unsigned char* vw = lds + wave * kVB;
  {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(V + kvoff * kD, (uint32_t)S * kRowB);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = 4 * i + (lane >> 4);
      dma16_buf(rs, (CA_LDS void*)(vw + 1024 * i),
                (uint32_t)(kw0 + row) * kRowB + 16 * ((lane & 15) ^ swz(row)));
    }
  }
  vec8 kv[8];  // K^T as the B operand of S = Q K^T (column = this lane's key)
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    if (kvalid) {
      kv[ks] = *(const vec8*)(K + (kvoff + mykey) * kD + 16 * ks + 8 * hl);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) kv[ks][e] = 0;
    }
  }

  const int t_begin = CAUSAL ? K0 / BQ : 0;
  const int nt = max(0, (S + BQ - 1) / BQ - t_begin);  // query tiles per q head
  const int n_it = G * nt;
  // ring load of tile it: one 1-KB load of Q and of dO per wave (tile rows
  // 4 wave + lane/16), the 64 floats of pairs by wave 0
  const int dma_row = 4 * wave + (lane >> 4);
  const uint32_t dma_off = dma_row * kRowB + 16 * ((lane & 15) ^ swz(dma_row));
  auto issue = [&](int it) CA_INLINE {
    unsigned char* st = lds + kNW * kVB + (it % kStages) * kStageB;
    // past the walk (slots the loop never reads): offsets past the slice, zeros
    const bool past = it >= n_it;
    const int itc = past ? 0 : it;
    const int h = hk * G + itc / max(nt, 1);
    const int q0 = past ? S : (t_begin + itc % max(nt, 1)) * BQ;
    const size_t ho = (size_t)(b * Hq + h) * S;
    const uint32_t qoff = (uint32_t)q0 * kRowB, sz = (uint32_t)S * kRowB;
    dma16_buf(make_rsrc_at(Q + ho * kD, qoff, sz), (CA_LDS void*)(st + 1024 * wave), dma_off);
    dma16_buf(make_rsrc_at(dO + ho * kD, qoff, sz), (CA_LDS void*)(st + kTileB + 1024 * wave),
              dma_off);
    if (wave == 0)
      dma4_buf(make_rsrc_at(LD + 2 * ho, (uint32_t)q0 * 8, (uint32_t)S * 8),
               (CA_LDS void*)(st + 2 * kTileB), 4 * lane);
  };
  const uint32_t lds0 = lds_off(lds);
  const uint32_t rofs = row_ofs(rho32(l32), hl);  // Q / dO rows (A operands)
  const uint32_t vofs = lds0 + wave * kVB + row_ofs(l32, hl);  // V rows (B operand)
  const TrOfs tofs = tr_ofs(lane);

  f32x16 dk[4], dv[4];  // dK^T, dV^T: rows d = 32 ob + .., column = this lane's key
#pragma unroll
  for (int i = 0; i < 4; ++i)
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
    if (CA_BWD_PRIO) __builtin_amdgcn_s_setprio(1);
    u32x4 qr[2], gr[2], vr[2];
    qr[0] = lds_read_b128<0>(qa);
    gr[0] = lds_read_b128<0>(ga);
    vr[0] = lds_read_b128<0>(vofs);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const int cb = ks & 1;
      if (ks < 7) {
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
    if (CA_BWD_PRIO) __builtin_amdgcn_s_setprio(0);
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
    if (CA_BWD_PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) {
      const vec8 g0 = tr_operand<Tr, 0>(sb + kTileB, tofs, ob);
      const vec8 g1 = tr_operand<Tr, 1>(sb + kTileB, tofs, ob);
      const vec8 x0 = tr_operand<Tr, 0>(sb, tofs, ob);
      const vec8 x1 = tr_operand<Tr, 1>(sb, tofs, ob);
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
    if (CA_BWD_PRIO) __builtin_amdgcn_s_setprio(0);
  };

#pragma unroll
  for (int i = 0; i < kDist; ++i) issue(i);
  for (int it = 0; it < n_it; ++it) {
    // this wave's loads of tile it (and its V rows, issued first) landed
    if (wave == 0) wait_vmcnt<3 * (kDist - 1)>();
    else wait_vmcnt<2 * (kDist - 1)>();
    __builtin_amdgcn_s_barrier();  // ... and every wave's; slot of it-1 is free
    issue(it + kDist);
    const int q0 = (t_begin + it % nt) * BQ;
    if (kw0 < S && (!CAUSAL || q0 >= kw0)) {  // causal: queries before every key of the wave
      const uint32_t sb = lds0 + kNW * kVB + (uint32_t)((it % kStages) * kStageB);
      tile(sb, q0, (CAUSAL && q0 == kw0) || q0 + BQ > S);
    }
  }
  wait_vmcnt<0>();  // no load may still target this workgroup's LDS when it exits
  if (kvalid) {
    const size_t koff = (kvoff + mykey) * kD;
    store_rowT<Tr, 4>(dK + koff, dk, hl, scale);
    store_rowT<Tr, 4>(dV + koff, dv, hl, 1.f);
  }
}

template <typename Tr, bool CAUSAL>
__global__ __launch_bounds__(64 * bw128::kNW) void bwd_dkv128_kernel(
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
    bwd_dkv128_tile<Tr, CAUSAL>(Q, K, V, dO, LD, dK, dV, S, Hq, Hkv, scale,
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
  const int n_qt = (S + 32 * kBwdWaves - 1) / (32 * kBwdWaves);
  const long long g1 = (long long)B * Hq * n_qt;
  const long long g2 = (long long)B * Hkv * n_qt;  // key tiles are as tall as query tiles
  if (g0 > 0x7fffffffLL || g1 > 0x7fffffffLL || g2 > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((bwd_rowdot_kernel<Tr, D>), dim3((unsigned)g0), dim3(256), 0, stream,
                     (const uint16_t*)o, (const uint16_t*)dout, lse, ws, rows);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (D == 128 && kBwdDma) {
    // 256 keys (dK, dV) / 256 queries (dQ) per workgroup, one workgroup per CU
    constexpr int BT = 32 * bw128::kNW;
    const int n_t = (S + BT - 1) / BT;
    int pk = 0, pq = 0;
    const long long gk = prefill_grid(B, Hkv, n_t, CAUSAL, 1, &pk);
    const long long gq = prefill_grid(B, Hq, n_t, CAUSAL, 1, &pq);
    if (gk > 0x7fffffffLL || gq > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL((bwd_dkv128_kernel<Tr, CAUSAL>), dim3((unsigned)gk), dim3(64 * bw128::kNW),
                       0, stream, (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,
                       (const uint16_t*)dout, ws, (uint16_t*)dk, (uint16_t*)dv, S, Hq, Hkv, scale,
                       n_t, B * Hkv, (int)gk, pk);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((bwd_dq128_kernel<Tr, CAUSAL>), dim3((unsigned)gq), dim3(64 * bw128::kNW),
                       0, stream, (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,
                       (const uint16_t*)dout, ws, (uint16_t*)dq, S, Hq, Hkv, scale, n_t, B * Hq,
                       (int)gq, pq);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((bwd_dkv_kernel<Tr, D, CAUSAL>), dim3((unsigned)g2), dim3(kBwdWaves * 64), 0,
                     stream, (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,
                     (const uint16_t*)dout, ws, (uint16_t*)dk, (uint16_t*)dv, S, Hq, Hkv, scale,
                     n_qt, (int)g2);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((bwd_dq_kernel<Tr, D, CAUSAL>), dim3((unsigned)g1), dim3(kBwdWaves * 64), 0,
                     stream, (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,
                     (const uint16_t*)dout, ws, (uint16_t*)dq, S, Hq, Hkv, scale, n_qt, (int)g1);
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
