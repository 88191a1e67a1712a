// Prefill (flash-attention forward) for gfx950: bf16/fp16 MFMA, K/V tiles in
// LDS, online softmax in registers.
//
// Computes O = softmax(Q K^T * scale [+ causal mask]) V per (batch, q-head),
// the contract of dispatch_flash_attention_v2 / _v3_hopper / fused_gqa in the
// reference (kernels_api.h:29-33,52-56,78-83; math flash_attention_v2_kernel.cuh:
// 82-83 causal tile bound, 179-229 online softmax, 223 l == 0 -> 0).
//
// Work decomposition
//   one workgroup = NW waves = BM = 32*NW query rows of one (b, h);
//   each wave owns 32 query rows for the whole KV walk;
//   KV tiles of BN = 64 keys are staged in LDS (double buffered, one barrier
//   per tile) and shared by the NW waves.
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
#include "common.h"
#include "launch.h"

namespace ca {

template <typename Tr, int D, int NW, bool CAUSAL>
__global__ __launch_bounds__(NW * 64, 2) void prefill_fwd_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, uint16_t* __restrict__ O, int S, int Hq,
    int Hkv, float scale_log2, int n_qt) {
  using vec8 = typename Tr::vec8;
  using vec4 = typename Tr::vec4;
  using vec2 = typename Tr::vec2;
  constexpr int BM = 32 * NW;
  constexpr int BN = 64;
  constexpr int KS = D + 8;    // K row stride (elements): permuted-row b128 reads hit distinct banks
  constexpr int VS = D + 32;   // V row stride: 4 consecutive rows land 64 B apart mod 256 B (tr16 reads)
  constexpr int NKS = D / 16;  // QK k-steps
  constexpr int NOB = D / 32;  // O^T row blocks
  constexpr int CHUNKS = D / 8;                 // 16-byte chunks per row
  constexpr int ROWS_PER_PASS = NW * 64 / CHUNKS;
  constexpr int PASSES = BN / ROWS_PER_PASS;
  static_assert(PASSES * ROWS_PER_PASS == BN, "tile staging must cover the tile");

  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][BN * KS];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][BN * VS];

  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = work / n_qt;
  const int qt = n_qt - 1 - (work % n_qt);  // longest causal tiles first
  const int b = bh / Hq, h = bh % Hq;
  const int hk = h / (Hq / Hkv);
  const int q0 = qt * BM;
  const uint16_t* Qp = Q + (size_t)(b * Hq + h) * S * D;
  uint16_t* Op = O + (size_t)(b * Hq + h) * S * D;
  const uint16_t* Kp = K + (size_t)(b * Hkv + hk) * S * D;
  const uint16_t* Vp = V + (size_t)(b * Hkv + hk) * S * D;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, hl = lane >> 5;
  const int qw0 = q0 + wave * 32;
  const int myq = qw0 + l32;

  // Q as the B operand of S^T = K Q^T: lane (q = l32, k-group hl)
  vec8 qv[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    if (myq < S) {
      qv[ks] = *(const vec8*)(Qp + (size_t)myq * D + 16 * ks + 8 * hl);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qv[ks][e] = 0;
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
      *(u32x4*)(&Vs[buf][r * VS + st_col]) = vreg[p];
    }
  };

  f32x16 o[NOB];
#pragma unroll
  for (int i = 0; i < NOB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
  float m_run = kNegInf, l_run = 0.f;

  const int krow = (l32 & 0x13) | ((l32 & 4) << 1) | ((l32 & 8) >> 1);
  // tr16 source-lane coordinates for the V^T operand
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
    f32x16 s[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) { s[0][r] = 0.f; s[1][r] = 0.f; }
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const vec8 a = *(const vec8*)(Kb + (32 * mb + krow) * KS + 16 * ks + 8 * hl);
        s[mb] = Tr::mfma32(a, qv[ks], s[mb]);
      }
    }

    // Softmax in the log2 domain with the scale folded into one FMA per
    // logit: p = 2^(s*c - m). The row max is taken over the raw logits (min
    // for a negative scale) and scaled once; a masked logit is set to the
    // value whose scaled image is -inf.
    const bool need_mask = CAUSAL ? (k0 + BN - 1 > qw0) : (k0 + BN > S);
    const bool pos = scale_log2 >= 0.f;
    if (need_mask) {
      const float mv = pos ? kNegInf : -kNegInf;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + 32 * mb + 16 * (r >> 3) + 8 * hl + (r & 7);
          const bool masked = (key >= S) || (CAUSAL && key > myq);
          if (masked) s[mb][r] = mv;
        }
    }
    float tm;
    if (pos) {
      tm = max3(s[0][0], s[0][1], s[0][2]);
#pragma unroll
      for (int i = 3; i < 31; i += 2) tm = max3(tm, s[i >> 4][i & 15], s[(i + 1) >> 4][(i + 1) & 15]);
      tm = __builtin_fmaxf(tm, s[1][15]);
    } else {
      tm = s[0][0];
#pragma unroll
      for (int i = 1; i < 32; ++i) tm = __builtin_fminf(tm, s[i >> 4][i & 15]);
    }
    float tmax = pair32_max(tm * scale_log2);
    const bool need = tmax > m_run + 8.0f;
    if (wave_any(need)) {
      const float m_new = __builtin_fmaxf(m_run, tmax);
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
    vec8 pb[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int base = (kk >> 1) * 16 + (kk & 1) * 8;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i0 = base + 2 * j, i1 = i0 + 1;
        const float p0 = fast_exp2(__builtin_fmaf(s[i0 >> 4][i0 & 15], scale_log2, -msub));
        const float p1 = fast_exp2(__builtin_fmaf(s[i1 >> 4][i1 & 15], scale_log2, -msub));
        psum += p0 + p1;
        const vec2 pk = Tr::pack2(p0, p1);
        pb[kk][2 * j] = pk[0];
        pb[kk][2 * j + 1] = pk[1];
      }
    }
    l_run += psum;

#pragma unroll
    for (int ob = 0; ob < NOB; ++ob) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const uint16_t* src = Vb + (16 * kk + tr_row) * VS + 32 * ob + tr_col;
        const vec4 lo = Tr::tr_read((const CA_LDS void*)src);
        const vec4 hi = Tr::tr_read((const CA_LDS void*)(src + 4 * VS));
        const vec8 a = cat4<vec8, vec4>(lo, hi);
        o[ob] = Tr::mfma32(a, pb[kk], o[ob]);
      }
    }
  }

  const float l_tot = pair32_sum(l_run);
  const float inv = (l_tot > 0.f) ? 1.f / l_tot : 0.f;
  if (myq < S) {
#pragma unroll
    for (int ob = 0; ob < NOB; ++ob) {
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

template <typename Tr, int D, bool CAUSAL>
static hipError_t launch_prefill_t(const void* q, const void* k, const void* v, void* o,
                                   int B, int Hq, int Hkv, int S, float scale,
                                   hipStream_t stream) {
#ifndef CA_PF_NW
#define CA_PF_NW 4
#endif
  constexpr int NW = CA_PF_NW;  // waves per workgroup (32 query rows each)
  constexpr int BM = 32 * NW;
  const int n_qt = (S + BM - 1) / BM;
  const long long grid = (long long)n_qt * B * Hq;
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL((prefill_fwd_kernel<Tr, D, NW, CAUSAL>), dim3((unsigned)grid),
                     dim3(NW * 64), 0, stream, (const uint16_t*)q, (const uint16_t*)k,
                     (const uint16_t*)v, (uint16_t*)o, S, Hq, Hkv, scale * kLog2e, n_qt);
  return hipGetLastError();
}

hipError_t launch_prefill(int dtype, const void* q, const void* k, const void* v, void* o,
                          int B, int Hq, int Hkv, int S, int D, float scale, bool causal,
                          hipStream_t stream) {
#define CA_PREFILL_CASE(TR, DD)                                                          \
  if (D == DD) {                                                                         \
    return causal ? launch_prefill_t<TR, DD, true>(q, k, v, o, B, Hq, Hkv, S, scale, stream) \
                  : launch_prefill_t<TR, DD, false>(q, k, v, o, B, Hq, Hkv, S, scale, stream); \
  }
  if (dtype == kDtypeBF16) {
    CA_PREFILL_CASE(BF16, 64)
    CA_PREFILL_CASE(BF16, 128)
  } else if (dtype == kDtypeF16) {
    CA_PREFILL_CASE(F16, 64)
    CA_PREFILL_CASE(F16, 128)
  }
#undef CA_PREFILL_CASE
  return hipErrorInvalidValue;
}

}  // namespace ca
