// MXFP8 attention for gfx950: q, k, v are OCP e4m3 codes [B, H, S, D] with one
// e8m0 scale byte per 32 consecutive elements along D ([B, H, S, D/32]).
//
// The reference declares the entry point (dispatch_fused_microscaled_attention,
// kernels_api.h:103-108; README.md:29-31,80-81) but ships no kernel; the
// semantics here are attention over the dequantised tensors
// x = code * 2^(scale - 127), fp32 accumulation, 16-bit output.
//
// QK^T contracts over D, the axis the MX blocks run along, so it maps onto
// v_mfma_scale_f32_32x32x64_f8f6f4: each MFMA covers 64 d (two MX blocks) and
// takes one e8m0 byte per lane. Hardware k-block 0 of that instruction is
// bytes 0-15 of both lane halves and block 1 bytes 16-31, with the scale of
// block b read from lane half b; so lane half h loads d = 64s + 16h + [0,16)
// into bytes 0-15 and d = 64s + 32 + 16h + [0,16) into bytes 16-31, and passes
// the scale of MX block 2s + h. The same assignment is used for A (K) and B
// (Q), so every fp8 product is paired with its own two scales.
//
// PV contracts over keys, while V's scales vary along D, so they cannot ride
// the MFMA scale operand: V is dequantised exactly into bf16 (e4m3 * 2^e is a
// bf16 value) while it is staged into LDS, and PV runs on bf16 MFMAs with P in
// bf16, as in the bf16 prefill kernel (same transposed S/O layout, same key
// permutation, same lazy online softmax).
#include "common.h"
#include "launch.h"

namespace ca {

__device__ __forceinline__ float e8m0_to_float(uint32_t e) {
  // 2^(e-127); e = 0 is the fp32 subnormal 2^-127, e = 255 is NaN
  if (e == 0) return __uint_as_float(0x00400000u);
  if (e == 255) return __uint_as_float(0x7fc00000u);
  return __uint_as_float(e << 23);
}

// One query tile (BM rows of head bh): the key walk and the output store.
// Other waves may still read the LDS tiles when a wave returns.
template <typename Tr, bool CAUSAL>
__device__ CA_INLINE void mxfp8_qtile(
    const uint8_t* __restrict__ Q, const uint8_t* __restrict__ QS, const uint8_t* __restrict__ K,
    const uint8_t* __restrict__ KSc, const uint8_t* __restrict__ V, const uint8_t* __restrict__ VSc,
    uint16_t* __restrict__ O, int S, float scale_log2, int bh, int qt) {
  using vec8 = BF16::vec8;
  using vec4 = BF16::vec4;
  using vec2 = BF16::vec2;
  constexpr int D = 128;
  constexpr int NW = 4;
  constexpr int BM = 32 * NW;
  constexpr int BN = 64;
  constexpr int NB = D / 32;   // MX blocks per row
  constexpr int KSB = D + 16;  // K byte row stride
  constexpr int VS = D + 32;   // V bf16 row stride (elements)
  constexpr int NOB = D / 32;

  __shared__ __attribute__((aligned(16))) uint8_t Ks[2][BN * KSB];
  __shared__ __attribute__((aligned(16))) uint32_t Kscl[2][BN];  // 4 e8m0 bytes per key
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][BN * VS];

  const int q0 = qt * BM;
  const size_t base = (size_t)bh * S;
  const uint8_t* Qp = Q + base * D;
  const uint8_t* Kp = K + base * D;
  const uint8_t* Vp = V + base * D;
  const uint8_t* QSp = QS + base * NB;
  const uint8_t* KSp = KSc + base * NB;
  const uint8_t* VSp = VSc + base * NB;
  uint16_t* Op = O + base * D;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, hl = lane >> 5;
  const int qw0 = q0 + wave * 32;
  const int myq = qw0 + l32;

  // Q operand (B of the scaled MFMA) and its scale bytes
  i32x8 qv[2];
  int qsc[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    if (myq < S) {
      const u32x4 lo = *(const u32x4*)(Qp + (size_t)myq * D + 64 * s + 16 * hl);
      const u32x4 hi = *(const u32x4*)(Qp + (size_t)myq * D + 64 * s + 32 + 16 * hl);
      qv[s] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      qsc[s] = QSp[(size_t)myq * NB + 2 * s + hl];
    } else {
      qv[s] = i32x8{0, 0, 0, 0, 0, 0, 0, 0};
      qsc[s] = 127;
    }
  }

  const int kv_end = CAUSAL ? min(S, q0 + BM) : S;
  const int n_tiles = (kv_end + BN - 1) / BN;

  // staging: 64 rows x 128 B per tile for K and V: thread -> (row, 16-byte chunk), 2 passes
  const int st_row = tid >> 3, st_ch = tid & 7;
  u32x4 kreg[2], vreg[2];
  uint32_t ksreg = 0, vsreg[2];
  auto gload = [&](int t) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int row = t * BN + st_row + 32 * p;
      if (row < S) {
        kreg[p] = *(const u32x4*)(Kp + (size_t)row * D + 16 * st_ch);
        vreg[p] = *(const u32x4*)(Vp + (size_t)row * D + 16 * st_ch);
        vsreg[p] = VSp[(size_t)row * NB + (st_ch >> 1)];
      } else {
        kreg[p] = u32x4{0, 0, 0, 0};
        vreg[p] = u32x4{0, 0, 0, 0};
        vsreg[p] = 127;
      }
    }
    if (tid < BN) {
      const int row = t * BN + tid;
      ksreg = (row < S) ? *(const uint32_t*)(KSp + (size_t)row * NB) : 0x7f7f7f7fu;
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int r = st_row + 32 * p;
      *(u32x4*)(&Ks[buf][r * KSB + 16 * st_ch]) = kreg[p];
      const float sc = e8m0_to_float(vsreg[p]);
      vec8 a, b;
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const bf16x2 c0 = e4m3x2_to_bf16_scaled<false>(vreg[p][w], sc);
        const bf16x2 c1 = e4m3x2_to_bf16_scaled<true>(vreg[p][w], sc);
        a[4 * w] = c0[0]; a[4 * w + 1] = c0[1]; a[4 * w + 2] = c1[0]; a[4 * w + 3] = c1[1];
        const bf16x2 c2 = e4m3x2_to_bf16_scaled<false>(vreg[p][2 + w], sc);
        const bf16x2 c3 = e4m3x2_to_bf16_scaled<true>(vreg[p][2 + w], sc);
        b[4 * w] = c2[0]; b[4 * w + 1] = c2[1]; b[4 * w + 2] = c3[0]; b[4 * w + 3] = c3[1];
      }
      *(vec8*)(&Vs[buf][r * VS + 16 * st_ch]) = a;
      *(vec8*)(&Vs[buf][r * VS + 16 * st_ch + 8]) = b;
    }
    if (tid < BN) Kscl[buf][tid] = ksreg;
  };

  f32x16 o[NOB];
#pragma unroll
  for (int i = 0; i < NOB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
  float m_run = kNegInf, l_run = 0.f;

  const int krow = (l32 & 0x13) | ((l32 & 4) << 1) | ((l32 & 8) >> 1);
  const int g16 = lane >> 4, s16 = lane & 15;
  const int tr_row = 8 * (g16 >> 1) + (s16 >> 2);
  const int tr_col = 16 * (g16 & 1) + 4 * (s16 & 3);

  // One key tile. The wave's first tile (t = 0, never skipped) takes the row
  // max; later tiles take their exponentials against the running max as it
  // stands, and only a tile whose bf16 weights sum past 2^48 in some lane
  // (or overflow) recomputes them after a full max and rescale: the weights
  // may exceed 1 by far while they stay representable in bf16 and O, l far
  // below the float range.
  auto step = [&](int t, auto first_tag) CA_INLINE {
    constexpr bool FIRST = decltype(first_tag)::value;
    const int buf = t & 1;
    lstore(buf);
    __syncthreads();
    if (t + 1 < n_tiles) gload(t + 1);
    const int k0 = t * BN;
    if (CAUSAL && k0 > qw0 + 31) return;

    f32x16 s[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) { s[0][r] = 0.f; s[1][r] = 0.f; }
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int row = 32 * mb + krow;
      const uint32_t ksw = Kscl[buf][row];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const u32x4 lo = *(const u32x4*)(&Ks[buf][row * KSB + 64 * st + 16 * hl]);
        const u32x4 hi = *(const u32x4*)(&Ks[buf][row * KSB + 64 * st + 32 + 16 * hl]);
        const i32x8 a = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        const int ksc = (ksw >> (8 * (2 * st + hl))) & 0xff;
        s[mb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, qv[st], s[mb], 0, 0, 0, ksc, 0, qsc[st]);
      }
    }
    // (the MFMA blocks run at raised wave priority: a wave's MFMAs then win
    // issue over the other waves' softmax VALU)
    __builtin_amdgcn_s_setprio(0);

    // masked logits (bounds, causal diagonal) become the value whose scaled
    // image is -inf, once, on the tiles that need it
    if (CAUSAL ? (k0 + BN - 1 > qw0) : (k0 + BN > S)) {
      const float mask_s = scale_log2 >= 0.f ? kNegInf : -kNegInf;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int key = k0 + 32 * (i >> 4) + 16 * ((i >> 3) & 1) + 8 * hl + (i & 7);
        if ((key >= S) || (CAUSAL && key > myq)) s[i >> 4][i & 15] = mask_s;
      }
    }
    // the tile's row max (log2 units) into the running max; O and l rescaled
    auto full_max = [&]() CA_INLINE {
      float tmax = kNegInf;
#pragma unroll
      for (int i = 0; i < 32; ++i) tmax = __builtin_fmaxf(tmax, s[i >> 4][i & 15] * scale_log2);
      tmax = pair32_max(tmax);
      if (wave_any(tmax > m_run + 8.0f)) {
        const float m_new = __builtin_fmaxf(m_run, tmax);
        const float alpha = (m_new == kNegInf) ? 1.f : fast_exp2(m_run - m_new);
#pragma unroll
        for (int i = 0; i < NOB; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
        l_run *= alpha;
        m_run = m_new;
      }
    };
    float psum = 0.f;
    vec8 pb[4];
    // P = 2^(s scale_log2 - m) as the PV B operand; the row sum uses the
    // bf16-rounded weights that enter PV (one dot2 with ones per pair), so
    // o / l is an exact weighted mean of V under slightly perturbed weights:
    // with MX data |v| reaches ~16 and the unrounded sum would put the P
    // rounding error (up to 2^-9 relative) straight into |o|
    auto weights = [&]() CA_INLINE {
      const float msub = (m_run == kNegInf) ? 0.f : m_run;
      const bf16x2 ones = {(__bf16)1.f, (__bf16)1.f};
      psum = 0.f;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i0 = (kk >> 1) * 16 + (kk & 1) * 8 + 2 * j;
          const float p0 = fast_exp2(__builtin_fmaf(s[i0 >> 4][i0 & 15], scale_log2, -msub));
          const float p1 = fast_exp2(__builtin_fmaf(s[(i0 + 1) >> 4][(i0 + 1) & 15], scale_log2, -msub));
          const vec2 pk = BF16::pack2(p0, p1);
          psum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pk), ones, psum, false);
          pb[kk][2 * j] = pk[0];
          pb[kk][2 * j + 1] = pk[1];
        }
      }
    };
    if (FIRST) {
      full_max();
      weights();
    } else {
      weights();
      if (__builtin_expect(wave_any(!(psum <= 0x1p48f)), 0)) {
        full_max();
        weights();
      }
    }
    l_run += psum;

    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ob = 0; ob < NOB; ++ob) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const uint16_t* src = &Vs[buf][(16 * kk + tr_row) * VS + 32 * ob + tr_col];
        const vec4 lo = BF16::tr_read((const CA_LDS void*)src);
        const vec4 hi = BF16::tr_read((const CA_LDS void*)(src + 4 * VS));
        o[ob] = BF16::mfma32(cat4<vec8, vec4>(lo, hi), pb[kk], o[ob]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };
  if (n_tiles > 0) {
    gload(0);
    step(0, std::true_type{});
  }
  for (int t = 1; t < n_tiles; ++t) step(t, std::false_type{});

  const float l_tot = pair32_sum(l_run);
  const float inv = (l_tot > 0.f) ? 1.f / l_tot : 0.f;
  if (myq < S) {
    using ovec4 = typename Tr::vec4;
    using ovec2 = typename Tr::vec2;
#pragma unroll
    for (int ob = 0; ob < NOB; ++ob) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d = 32 * ob + 8 * a + 4 * hl;
        const ovec2 lo = Tr::pack2(o[ob][4 * a] * inv, o[ob][4 * a + 1] * inv);
        const ovec2 hi = Tr::pack2(o[ob][4 * a + 2] * inv, o[ob][4 * a + 3] * inv);
        ovec4 w;
        w[0] = lo[0]; w[1] = lo[1]; w[2] = hi[0]; w[3] = hi[1];
        *(ovec4*)(Op + (size_t)myq * D + d) = w;
      }
    }
  }
}

template <typename Tr, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void mxfp8_fwd_kernel(
    const uint8_t* __restrict__ Q, const uint8_t* __restrict__ QS, const uint8_t* __restrict__ K,
    const uint8_t* __restrict__ KSc, const uint8_t* __restrict__ V, const uint8_t* __restrict__ VSc,
    uint16_t* __restrict__ O, int S, float scale_log2, int n_qt, int n_bh, int n_work,
    int paired) {
  const QTileWork wk = prefill_work(xcd_remap(blockIdx.x, n_work), n_qt, n_bh, paired);
  const int n_pass = wk.qt1 < 0 ? 1 : 2;
#pragma clang loop unroll(disable)
  for (int pass = 0; pass < n_pass; ++pass) {
    // the second tile restages the LDS buffers: every wave must be done reading them
    if (pass) __syncthreads();
    mxfp8_qtile<Tr, CAUSAL>(Q, QS, K, KSc, V, VSc, O, S, scale_log2, pass ? wk.bh1 : wk.bh0,
                            pass ? wk.qt1 : wk.qt0);
  }
}

hipError_t launch_mxfp8(int out_dtype, const uint8_t* q, const uint8_t* qs, const uint8_t* k,
                        const uint8_t* ks, const uint8_t* v, const uint8_t* vs, void* o, int B,
                        int H, int S, int D, float scale, bool causal, hipStream_t stream) {
  if (D != 128) return hipErrorInvalidValue;
  constexpr int BM = 128;
  const int n_qt = (S + BM - 1) / BM;
  int paired = 0;
  const long long grid = prefill_grid(B, H, n_qt, causal, 2, &paired);
  if (grid == 0) return hipSuccess;
  if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
  const float sl2 = scale * kLog2e;
#define CA_MX(TR, C)                                                                         \
  hipLaunchKernelGGL((mxfp8_fwd_kernel<TR, C>), dim3((unsigned)grid), dim3(256), 0, stream, q, \
                     qs, k, ks, v, vs, (uint16_t*)o, S, sl2, n_qt, B * H, (int)grid, paired);
  if (out_dtype == kDtypeBF16) {
    if (causal) { CA_MX(BF16, true) } else { CA_MX(BF16, false) }
  } else if (out_dtype == kDtypeF16) {
    if (causal) { CA_MX(F16, true) } else { CA_MX(F16, false) }
  } else {
    return hipErrorInvalidValue;
  }
#undef CA_MX
  return hipGetLastError();
}

}  // namespace ca
