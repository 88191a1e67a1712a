// float32 prefill (flash-attention forward) for gfx950 on fp32 MFMAs.
//
// The reference instantiates its prefill entry points for float
// (flash_attention_v2_instantiations.cu, flash_attention_v3_hopper_
// instantiations.cu, fused_gqa_instantiations.cu; binding
// fused_softmax_binding.cpp:77-81). Same contract as the 16-bit kernels:
// O = softmax(Q K^T * scale [+ causal mask]) V per (b, q head), GQA by
// kv_head = q_head / (Hq / Hkv), O = 0 for a row with no visible key.
//
// Two kernels. prefill_f32_kernel: one workgroup = 4 waves x 32 query rows of
// one (b, h); K/V tiles of 32 keys, double-buffered in LDS (register-staged
// loads, one barrier per tile). prefill_f32_split_kernel (launches with fewer
// 128-row tiles than CUs): one workgroup per pair of 32-row query blocks, its
// 4 waves splitting the pair's key tiles and merging their softmax states
// (described at the kernel). Per wave and tile, both on
// v_mfma_f32_32x32x2_f32 (one fp32 element of each operand per lane,
// k = lane / 32):
//   S^T[32 keys x 32 q] = K Q^T   over D/2 steps; lane half h contracts
//     head-dim elements (D/2) h + step (the split kernel: 8 j + 4 h + c at
//     step 4 j + c), so a lane's K row and Q row are read as float4s;
//   O^T[D x 32 q] += V^T P^T       over 16 steps of two keys.
// Key permutation: accumulator register r of lane half h holds S^T row
// 8 (r/4) + 4 h + r%4 (the 32x32 accumulator layout); the A-operand lane for
// that row reads key 16 h + r, so register r of half h is exactly the PV
// B-operand element for key 16 h + r at step r: P never leaves its registers.
// LDS (prefill_f32_kernel): K row-major with row stride D + 4 floats, V
// transposed ([D][32 keys]) with row stride 36 floats; both make the float4
// operand reads of a 16-lane group hit 16 distinct 4-bank groups.
#include "common.h"
#include "launch.h"

namespace ca {

// One query tile (BM rows of head bh): the key walk and the output store.
// Other waves may still read the LDS tiles when a wave returns.
template <int D, bool CAUSAL>
__device__ CA_INLINE void prefill_f32_qtile(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ Lse, int S, int Hq, int Hkv, float scale_log2, int bh, int qt) {
  constexpr int NW = 4;
  constexpr int BM = 32 * NW;
  constexpr int BN = 32;
  constexpr int KS = D + 4;     // K row stride (floats)
  constexpr int VS = BN + 4;    // V^T row stride (floats)
  constexpr int HD = D / 2;     // S^T contraction steps
  constexpr int NOB = D / 32;   // O^T row blocks
  constexpr int F4_ROW = D / 4;                  // float4s per K/V row
  constexpr int F4_TILE = BN * F4_ROW;           // float4s per tile
  constexpr int F4_PER_THREAD = F4_TILE / (NW * 64);
  static_assert(F4_PER_THREAD * NW * 64 == F4_TILE, "tile staging must cover the tile");

  __shared__ __attribute__((aligned(16))) float Ks[2][BN * KS];
  __shared__ __attribute__((aligned(16))) float Vt[2][D * VS];

  const int b = bh / Hq, h = bh % Hq;
  const int hk = h / (Hq / Hkv);
  const int q0 = qt * BM;
  const float* Qp = Q + (size_t)(b * Hq + h) * S * D;
  float* Op = O + (size_t)(b * Hq + h) * S * D;
  const float* Kp = K + (size_t)(b * Hkv + hk) * S * D;
  const float* Vp = V + (size_t)(b * Hkv + hk) * S * D;

  // lane recomputed per query tile (lane_here): hoisted out of the kernel's
  // pass loop, its offsets spilled at D = 128
  const int lane = lane_here();
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int tid = wave * 64 + lane;
  const int l32 = lane & 31, hl = lane >> 5;
  const int qw0 = q0 + wave * 32;
  const int myq = qw0 + l32;

  // Q as the B operand: qv[k] = Q[myq][HD * hl + k]
  float qv[HD];
#pragma unroll
  for (int k4 = 0; k4 < HD; k4 += 4) {
    float4 x = {0.f, 0.f, 0.f, 0.f};
    if (myq < S) x = *(const float4*)(Qp + (size_t)myq * D + HD * hl + k4);
    qv[k4] = x.x; qv[k4 + 1] = x.y; qv[k4 + 2] = x.z; qv[k4 + 3] = x.w;
  }

  const int kv_end = CAUSAL ? min(S, q0 + BM) : S;
  const int n_tiles = (kv_end + BN - 1) / BN;

  float4 kreg[F4_PER_THREAD], vreg[F4_PER_THREAD];
  auto gload = [&](int t) {
#pragma unroll
    for (int it = 0; it < F4_PER_THREAD; ++it) {
      const int idx = tid + NW * 64 * it;
      const int row = idx / F4_ROW, c4 = idx % F4_ROW;
      const int key = t * BN + row;
      if (key < S) {
        kreg[it] = *(const float4*)(Kp + (size_t)key * D + 4 * c4);
        vreg[it] = *(const float4*)(Vp + (size_t)key * D + 4 * c4);
      } else {
        kreg[it] = float4{0.f, 0.f, 0.f, 0.f};
        vreg[it] = float4{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int it = 0; it < F4_PER_THREAD; ++it) {
      const int idx = tid + NW * 64 * it;
      const int row = idx / F4_ROW, c4 = idx % F4_ROW;
      *(float4*)(&Ks[buf][row * KS + 4 * c4]) = kreg[it];
      float* vt = &Vt[buf][(4 * c4) * VS + row];
      vt[0] = vreg[it].x;
      vt[VS] = vreg[it].y;
      vt[2 * VS] = vreg[it].z;
      vt[3 * VS] = vreg[it].w;
    }
  };

  f32x16 o[NOB];
#pragma unroll
  for (int i = 0; i < NOB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
  float m_run = kNegInf, l_run = 0.f;
  const int krow = 16 * ((l32 >> 2) & 1) + 4 * (l32 >> 3) + (l32 & 3);

  if (n_tiles > 0) gload(0);
  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    lstore(buf);
    __syncthreads();
    if (t + 1 < n_tiles) gload(t + 1);
    const int k0 = t * BN;
    if (CAUSAL && k0 > qw0 + 31) continue;  // tile entirely above this wave's rows

    f32x16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
    const float* kr = Ks[buf] + krow * KS + HD * hl;
#pragma unroll
    for (int k4 = 0; k4 < HD; k4 += 4) {
      const float4 a = *(const float4*)(kr + k4);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, qv[k4], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, qv[k4 + 1], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, qv[k4 + 2], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, qv[k4 + 3], s, 0, 0, 0);
    }

    // online softmax in the log2 domain; register r holds key k0 + 16 hl + r
    float x[16];
    float tm = kNegInf;
    const bool need_mask = CAUSAL ? (k0 + BN - 1 > qw0) : (k0 + BN > S);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      x[r] = s[r] * scale_log2;
      if (need_mask) {
        const int key = k0 + 16 * hl + r;
        if (key >= S || (CAUSAL && key > myq)) x[r] = kNegInf;
      }
      tm = __builtin_fmaxf(tm, x[r]);
    }
    const float m_new = __builtin_fmaxf(m_run, pair32_max(tm));
    const float alpha = (m_new == kNegInf) ? 1.f : fast_exp2(m_run - m_new);
#pragma unroll
    for (int i = 0; i < NOB; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
    m_run = m_new;
    const float msub = (m_run == kNegInf) ? 0.f : m_run;
    float p[16];
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      p[r] = fast_exp2(x[r] - msub);
      psum += p[r];
    }
    l_run = l_run * alpha + psum;

    // O^T += V^T P^T: A = V^T[32 ob + l32][16 hl + step], B = p[step]
#pragma unroll
    for (int ob = 0; ob < NOB; ++ob) {
      const float* vr = Vt[buf] + (32 * ob + l32) * VS + 16 * hl;
#pragma unroll
      for (int k4 = 0; k4 < 16; k4 += 4) {
        const float4 a = *(const float4*)(vr + k4);
        o[ob] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, p[k4], o[ob], 0, 0, 0);
        o[ob] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, p[k4 + 1], o[ob], 0, 0, 0);
        o[ob] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, p[k4 + 2], o[ob], 0, 0, 0);
        o[ob] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, p[k4 + 3], o[ob], 0, 0, 0);
      }
    }
  }

  const float l_tot = pair32_sum(l_run);
  const float inv = (l_tot > 0.f) ? 1.f / l_tot : 0.f;
  if (Lse && hl == 0 && myq < S) Lse[(size_t)(b * Hq + h) * S + myq] = row_lse(m_run, l_tot);
  if (myq < S) {
#pragma unroll
    for (int ob = 0; ob < NOB; ++ob) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d = 32 * ob + 8 * a + 4 * hl;
        const float4 w = {o[ob][4 * a] * inv, o[ob][4 * a + 1] * inv, o[ob][4 * a + 2] * inv,
                          o[ob][4 * a + 3] * inv};
        *(float4*)(Op + (size_t)myq * D + d) = w;
      }
    }
  }
}

template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void prefill_f32_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ Lse, int S, int Hq, int Hkv, float scale_log2, int n_qt, int n_bh,
    int n_work, int paired) {
  const QTileWork wk = prefill_work(xcd_remap(blockIdx.x, n_work), n_qt, n_bh, paired);
  const int n_pass = wk.qt1 < 0 ? 1 : 2;
#pragma clang loop unroll(disable)
  for (int pass = 0; pass < n_pass; ++pass) {
    // the second tile restages the LDS buffers: every wave must be done reading them
    if (pass) __syncthreads();
    prefill_f32_qtile<D, CAUSAL>(Q, K, V, O, Lse, S, Hq, Hkv, scale_log2, pass ? wk.bh1 : wk.bh0,
                                 pass ? wk.qt1 : wk.qt0);
  }
}

// ---------------------------------------------------------------------------
// Small grids: the key walk of one 32-row query block split over the waves
// of a workgroup.
//
// When (b, h) x 128-row tiles would not give every CU a workgroup (BASELINE
// C1: 16 heads x 8 tiles = 128 workgroups on 256 CUs, the longest walking 32
// key tiles on each SIMD), a workgroup takes one 32-row query block and its
// four waves (one per SIMD) take key tiles w, w + 4, ... of it, each with its
// own online-softmax state; the states are merged through LDS at the end (O =
// sum_w a_w O_w / sum_w a_w l_w with a_w = 2^(m_w - max m)). Causal launches
// give a workgroup blocks p and n_qb-1-p (their walks add up to n_qb + 1 tiles
// for every p), non-causal launches with more blocks than CUs blocks p and
// p + n_qb/2, as one list of tiles dealt round-robin, so the waves stay within
// one tile of each other, and a wave goes on from its last tile of the first
// block to its first of the second without waiting for the others: each block
// has its own LDS region for the states, and one barrier precedes the merge
// of both.
//
// No wave shares a tile, so there is nothing to stage: every lane loads its
// MFMA operands straight from global memory (L2) into registers. S^T = K Q^T
// needs K row 16 h' + r (the key permutation above); lane half h contracts
// head-dim elements 8 j + 4 h + c at step 4 j + c, so the two halves of a
// float4 load read 32 adjacent bytes of a row (D/8 loads per tile);
// O^T += V^T P^T needs V[key 16 h + step][32 ob + l32]: one dword per lane and
// step, 32 lanes reading one 128-byte row segment.
//
// Measured on gfx950 (one wave per SIMD): a wave's VALU and memory
// instructions issue between its own fp32 MFMAs, not beside them (16 FMAs
// between two v_mfma_f32_32x32x2_f32 take 64 + ~77 cycles; a 16-byte load with
// the CU's four waves loading, ~60), and a second wave on the SIMD recovers
// little of that. So the tile time is MFMA time plus the wave's own VALU and
// load time: the walk keeps both small (no AGPR copies, masks and rescales
// only where needed, full-tile V loads from one address) rather than trying to
// hide them. Per 32-key tile at D = 64: 4096 MFMA cycles, ~5.3k measured.
// ---------------------------------------------------------------------------
template <int D>
struct SplitStage {
  static constexpr int NW = 4;      // waves per workgroup
  static constexpr int OS = D + 4;  // row stride (floats) of a wave's O block
  float o[2][NW][32 * OS];          // [block][wave]: unnormalised O rows
  float m[2][NW][32];               // row reference max m, log2 units (-inf: no tile)
  float l[2][NW][32];               // row sum of 2^(x - m)
};

// This wave's share of the key walks of query blocks qa and (qb2 >= 0) qb2:
// items g = wave, wave + NW, ... of the list [qa's tiles, qb2's tiles]; the
// state of each block goes to its stage region (zeros, -inf and 0 for a block
// in which the wave has no tile). The next item's K is loaded once this
// item's S MFMAs have read K, its V once the PV MFMAs have read V, and at the
// switch from block qa to qb2 the new Q once the last S MFMAs of qa have read
// Q, so the walk runs on from one block into the other.
template <int D, bool CAUSAL>
__device__ CA_INLINE void prefill_f32_split_walk(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V, int S,
    int Hq, int Hkv, float scale_log2, int bh, int qa, int qb2, SplitStage<D>& stg) {
  constexpr int HD = D / 2;
  constexpr int NOB = D / 32;
  constexpr int NW = SplitStage<D>::NW;
  constexpr int OS = SplitStage<D>::OS;

  const int b = bh / Hq, h = bh % Hq;
  const int hk = h / (Hq / Hkv);
  const float* Qp = Q + (size_t)(b * Hq + h) * S * D;
  const float* Kp = K + (size_t)(b * Hkv + hk) * S * D;
  const float* Vp = V + (size_t)(b * Hkv + hk) * S * D;

  const int tid = threadIdx.x;
  // wave index made scalar: the item loop and its branches are uniform
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int l32 = lane & 31, hl = lane >> 5;
  const int krow = 16 * ((l32 >> 2) & 1) + 4 * (l32 >> 3) + (l32 & 3);

  auto n_tiles_of = [&](int qb) { return CAUSAL ? qb + 1 : (S + 31) / 32; };
  const int na = n_tiles_of(qa);
  const int n_all = na + (qb2 >= 0 ? n_tiles_of(qb2) : 0);
  // item -> first key of its tile (items past the list clamp to valid rows)
  auto key0 = [&](int g) { return (g < na ? g : g - na) * 32; };

  f32x16 o[NOB];
  float m_run, l_run;
  auto reset = [&]() {
#pragma unroll
    for (int i = 0; i < NOB; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
    m_run = kNegInf;
    l_run = 0.f;
  };
  auto put_state = [&](int blk) {
    const float l_tot = pair32_sum(l_run);
    float* ow = stg.o[blk][wave] + l32 * OS;
#pragma unroll
    for (int ob = 0; ob < NOB; ++ob)
#pragma unroll
      for (int a = 0; a < 4; ++a)
        *(float4*)(ow + 32 * ob + 8 * a + 4 * hl) =
            float4{o[ob][4 * a], o[ob][4 * a + 1], o[ob][4 * a + 2], o[ob][4 * a + 3]};
    if (hl == 0) {
      stg.m[blk][wave][l32] = m_run;
      stg.l[blk][wave][l32] = l_tot;
    }
  };
  reset();

  int g = wave;
  if (g >= n_all) {
    put_state(0);
    if (qb2 >= 0) put_state(1);
    return;
  }
  if (g >= na) put_state(0);  // no tile of block qa

  // Q as the B operand; lane half h contracts head-dim elements 8 j + 4 h + c
  // at step 4 j + c, so the two halves of a float4 K load read 32 adjacent
  // bytes of a row
  float qv[HD];
  auto load_q = [&](float (&dst)[HD], int qb) {
    const int row = qb * 32 + l32;
#pragma unroll
    for (int k4 = 0; k4 < HD; k4 += 4) {
      float4 x = {0.f, 0.f, 0.f, 0.f};
      if (row < S) x = *(const float4*)(Qp + (size_t)row * D + 2 * k4 + 4 * hl);
      dst[k4] = x.x * scale_log2;
      dst[k4 + 1] = x.y * scale_log2;
      dst[k4 + 2] = x.z * scale_log2;
      dst[k4 + 3] = x.w * scale_log2;
    }
  };
  load_q(qv, g < na ? qa : qb2);

  // key rows past S are clamped to S - 1 (finite data; their logits are masked)
  float4 kr[HD / 4];
  float vr[NOB][16];
  auto load_k = [&](int gi) {
    const float* kp = Kp + (size_t)min(key0(gi) + krow, S - 1) * D + 4 * hl;
#pragma unroll
    for (int j = 0; j < HD / 4; ++j) kr[j] = *(const float4*)(kp + 8 * j);
  };
  auto load_v = [&](int gi) {
    const int k0 = key0(gi);
    if (k0 + 32 <= S) {  // whole tile: one address, immediate offsets
      const float* vp = Vp + (size_t)(k0 + 16 * hl) * D + l32;
#pragma unroll
      for (int st = 0; st < 16; ++st)
#pragma unroll
        for (int ob = 0; ob < NOB; ++ob) vr[ob][st] = vp[st * D + 32 * ob];
    } else {
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const float* vp = Vp + (size_t)min(k0 + 16 * hl + st, S - 1) * D + l32;
#pragma unroll
        for (int ob = 0; ob < NOB; ++ob) vr[ob][st] = vp[32 * ob];
      }
    }
  };
  auto qk = [&](f32x16& s) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
    for (int j = 0; j < HD / 4; ++j) {
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kr[j].x, qv[4 * j], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kr[j].y, qv[4 * j + 1], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kr[j].z, qv[4 * j + 2], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kr[j].w, qv[4 * j + 3], s, 0, 0, 0);
    }
  };
  // Online softmax of item gi in the log2 domain (Q carries the scale;
  // register r holds key k0 + 16 hl + r). A wave's VALU instructions issue
  // between its own MFMAs, not beside them, so every one of them lengthens the
  // tile: masks are applied only on a diagonal or ragged tile, and the running
  // max m is raised (and O, l rescaled) only when some row's tile max exceeds
  // it by more than 8, so p = 2^(x - m) <= 256 and most tiles skip the rescale.
  float p[16];
  auto softmax = [&](f32x16& s, int gi) {
    const int q0 = (gi < na ? qa : qb2) * 32;
    const int k0 = key0(gi);
    if ((CAUSAL && k0 == q0) || k0 + 32 > S) {
      const int lim = CAUSAL ? min(q0 + l32, S - 1) : S - 1;  // last visible key of this row
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (k0 + 16 * hl + r > lim) s[r] = kNegInf;
    }
    float tm = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) tm = __builtin_fmaxf(tm, s[r]);
    tm = pair32_max(tm);
    if (wave_any(tm > m_run + 8.f)) {
      const float m_new = __builtin_fmaxf(m_run, tm);
      const float alpha = (m_new == kNegInf) ? 1.f : fast_exp2(m_run - m_new);
#pragma unroll
      for (int i = 0; i < NOB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
      l_run *= alpha;
      m_run = m_new;
    }
    const float msub = (m_run == kNegInf) ? 0.f : m_run;
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      p[r] = fast_exp2(s[r] - msub);
      psum += p[r];
    }
    l_run += psum;
  };
  auto pv = [&]() {
#pragma unroll
    for (int ob = 0; ob < NOB; ++ob)
#pragma unroll
      for (int st = 0; st < 16; ++st)
        o[ob] = __builtin_amdgcn_mfma_f32_32x32x2f32(vr[ob][st], p[st], o[ob], 0, 0, 0);
  };

  f32x16 s;
  // Start the waves a few hundred cycles apart: a wave's loads issue between
  // its own MFMAs, each taking its share of the CU's L1 path, and four waves
  // in lockstep issue their loads at the same time (a lone wave's 16-byte
  // loads go through about three times faster); offset, their load phases
  // fall into one another's MFMA phases (measured: C1 -4.5 %).
  if (wave == 1) __builtin_amdgcn_s_sleep(10);
  if (wave == 2) __builtin_amdgcn_s_sleep(20);
  if (wave == 3) __builtin_amdgcn_s_sleep(30);
  load_k(g);
  load_v(g);
#pragma clang loop unroll(disable)
  for (;; g += NW) {
    const bool more = g + NW < n_all;
    const bool switch_blk = g < na && g + NW >= na && more;  // next item is in block qb2
    qk(s);
    if (switch_blk) load_q(qv, qb2);
    if (more) load_k(g + NW);
    softmax(s, g);
    pv();
    if (!more) break;
    load_v(g + NW);
    if (switch_blk) {
      put_state(0);
      reset();
    }
  }
  put_state(g < na ? 0 : 1);
  if (qb2 >= 0 && g < na) {  // no tile of block qb2
    reset();
    put_state(1);
  }
}

// Merge of the NW wave states of stage region blk into the output rows of
// query block qb: thread -> row, D / (2 NW) consecutive columns.
template <int D>
__device__ CA_INLINE void prefill_f32_split_merge(float* __restrict__ O, float* __restrict__ Lse,
                                                  int S, int bh, int qb, int blk,
                                                  const SplitStage<D>& stg) {
  constexpr int NW = SplitStage<D>::NW;
  constexpr int OS = SplitStage<D>::OS;
  constexpr int TPR = 2 * NW;  // threads per row
  constexpr int CW = D / TPR;  // columns per thread
  static_assert(CW % 4 == 0, "float4 columns");
  const int tid = threadIdx.x;
  const int row = tid / TPR, c0 = (tid % TPR) * CW;
  float mw[NW], aw[NW];
  float M = kNegInf;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    mw[w] = stg.m[blk][w][row];
    M = __builtin_fmaxf(M, mw[w]);
  }
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    aw[w] = (mw[w] == kNegInf) ? 0.f : fast_exp2(mw[w] - M);
    L += aw[w] * stg.l[blk][w][row];
  }
  const float inv = (L > 0.f) ? 1.f / L : 0.f;
  const int q = qb * 32 + row;
  if (q >= S) return;
  float* Op = O + ((size_t)bh * S + q) * D;
#pragma unroll
  for (int j = 0; j < CW; j += 4) {
    float4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float4 x = *(const float4*)(stg.o[blk][w] + row * OS + c0 + j);
      acc.x += aw[w] * x.x;
      acc.y += aw[w] * x.y;
      acc.z += aw[w] * x.z;
      acc.w += aw[w] * x.w;
    }
    *(float4*)(Op + c0 + j) = float4{acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv};
  }
  if (Lse && tid % TPR == 0) Lse[(size_t)bh * S + q] = row_lse(M, L);
}

// One workgroup per work item of a (b, h): block p, or two blocks: causal
// p and n_qb-1-p (equal total walks); non-causal, when the launch has more
// blocks than CUs, p and p + per_head (one round of workgroups instead of
// two). per_head = work items per (b, h).
template <int D, bool CAUSAL>
__global__ __launch_bounds__(64 * SplitStage<D>::NW, 1) void prefill_f32_split_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ Lse, int S, int Hq, int Hkv, float scale_log2, int n_qb,
    int per_head, int n_work) {
  __shared__ __attribute__((aligned(16))) SplitStage<D> stg;
  const int item = xcd_remap(blockIdx.x, n_work);
  const int bh = item / per_head, p = item % per_head;
  int p2 = CAUSAL ? n_qb - 1 - p : p + per_head;
  if (p2 == p || p2 >= n_qb) p2 = -1;
  prefill_f32_split_walk<D, CAUSAL>(Q, K, V, S, Hq, Hkv, scale_log2, bh, p, p2, stg);
  __syncthreads();
  prefill_f32_split_merge<D>(O, Lse, S, bh, p, 0, stg);
  if (p2 >= 0) prefill_f32_split_merge<D>(O, Lse, S, bh, p2, 1, stg);
}

template <int D, bool CAUSAL>
static hipError_t launch_prefill_f32_t(const void* q, const void* k, const void* v, void* o, float* lse,
                                       int B, int Hq, int Hkv, int S, float scale,
                                       hipStream_t stream) {
  constexpr int BM = 128;
  const int n_qt = (S + BM - 1) / BM;
  int paired = 0;
  const long long grid = prefill_grid(B, Hq, n_qt, CAUSAL, 2, &paired);
  if (grid == 0) return hipSuccess;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  if (grid < device_cus()) {
    // fewer 128-row tiles than CUs: split each 32-row block's key walk
    const int n_qb = (S + 31) / 32;
    const bool two = CAUSAL || (long long)B * Hq * n_qb > device_cus();
    const int per_head = two ? (n_qb + 1) / 2 : n_qb;
    const long long grid_s = (long long)B * Hq * per_head;
    hipLaunchKernelGGL((prefill_f32_split_kernel<D, CAUSAL>), dim3((unsigned)grid_s),
                       dim3(64 * SplitStage<D>::NW), 0, stream, (const float*)q, (const float*)k, (const float*)v, (float*)o, lse, S,
                       Hq, Hkv, scale * kLog2e, n_qb, per_head, (int)grid_s);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((prefill_f32_kernel<D, CAUSAL>), dim3((unsigned)grid), dim3(256), 0, stream,
                     (const float*)q, (const float*)k, (const float*)v, (float*)o, lse, S, Hq, Hkv,
                     scale * kLog2e, n_qt, B * Hq, (int)grid, paired);
  return hipGetLastError();
}

hipError_t launch_prefill_f32(const void* q, const void* k, const void* v, void* o, float* lse, int B,
                              int Hq, int Hkv, int S, int D, float scale, bool causal,
                              hipStream_t stream) {
  if (D == 64)
    return causal ? launch_prefill_f32_t<64, true>(q, k, v, o, lse, B, Hq, Hkv, S, scale, stream)
                  : launch_prefill_f32_t<64, false>(q, k, v, o, lse, B, Hq, Hkv, S, scale, stream);
  if (D == 128)
    return causal ? launch_prefill_f32_t<128, true>(q, k, v, o, lse, B, Hq, Hkv, S, scale, stream)
                  : launch_prefill_f32_t<128, false>(q, k, v, o, lse, B, Hq, Hkv, S, scale, stream);
  return hipErrorInvalidValue;
}

}  // namespace ca
