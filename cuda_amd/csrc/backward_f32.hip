// float32 flash-attention backward for gfx950 on fp32 MFMAs.
//
// The reference instantiates its backward for float as well
// (flash_attention_bwd_instantiations.cu:4; binding fused_softmax_binding.cpp:
// 396). Same contract and math as the 16-bit kernels of backward.hip
// (flash_attention_bwd_kernel.cuh:9-19,96-214): from q, k, v, o, dO and the
// forward's natural-log LSE,
//   D_i = rowsum(dO * O),  P = exp(S * scale - LSE_i),  dS = P (dP - D_i),
//   dQ = scale * dS K,  dK = scale * dS^T Q,  dV = P^T dO,
// P = dS = 0 where masked (key > query when causal) or past S; GQA sums dK,
// dV over the q heads of a kv head. Three launches, no atomics.
//
// On v_mfma_f32_32x32x2_f32 (one fp32 element of each operand per lane,
// k = lane / 32), with the float32 forward's row permutation: the A-operand
// lane of output row m reads tile row krow(m) = 16 ((m/4) % 2) + 4 (m/8) +
// m % 4, so accumulator register r of lane half h holds tile row 16 h + r —
// exactly the B-operand element of step r of the next product (which
// contracts tile rows r and 16 + r). P and dS never leave their registers.
//   dq kernel  (4 waves x 32 queries, K/V tiles of 32 keys in LDS):
//     S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dS^T (K^T read as single
//     floats, 32 consecutive dims per half wave);
//   dkv kernel (4 waves x 32 keys, Q/dO tiles of 32 queries of every q head):
//     S = Q K^T, dP = dO V^T, dV^T += dO^T P, dK^T += Q^T dS.
// Rows are stored with stride D + 4 floats so the float4 row reads of a
// 16-lane group fall on distinct 4-bank groups.
#include "common.h"
#include "launch.h"

namespace ca {
namespace {

constexpr int kF32Waves = 4;
constexpr int kF32Tile = 32;

__device__ __forceinline__ int krow32(int l32) {
  return 16 * ((l32 >> 2) & 1) + 4 * (l32 >> 3) + (l32 & 3);
}

// (LSE log2 e, rowsum(dO * O)) per query row; D / 4 lanes per row.
template <int D>
__global__ __launch_bounds__(256) void bwd_rowdot_f32_kernel(const float* __restrict__ O,
                                                             const float* __restrict__ dO,
                                                             const float* __restrict__ LSE,
                                                             float* __restrict__ LD,
                                                             long long rows) {
  constexpr int L = D / 4;
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long row = t / L;
  const int c = (int)(t % L);
  float acc = 0.f;
  if (row < rows) {
    const float4 o = *(const float4*)(O + row * D + 4 * c);
    const float4 g = *(const float4*)(dO + row * D + 4 * c);
    acc = o.x * g.x + o.y * g.y + o.z * g.z + o.w * g.w;
  }
#pragma unroll
  for (int m = L / 2; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if (row < rows && c == 0) {
    LD[2 * row] = LSE[row] * kLog2e;
    LD[2 * row + 1] = acc;
  }
}

// Stage 32 rows of two [.., D] fp32 tensors into registers (rows past S as
// zeros), then into padded LDS tiles.
template <int D>
struct Stage2 {
  static constexpr int KS = D + 4;
  static constexpr int F4_ROW = D / 4;
  static constexpr int PER = kF32Tile * F4_ROW / (kF32Waves * 64);
  static_assert(PER * kF32Waves * 64 == kF32Tile * F4_ROW, "staging must cover the tile");
  float4 a[PER], b[PER];
  __device__ __forceinline__ void load(const float* A, const float* B, int r0, int S, int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = tid + kF32Waves * 64 * i;
      const int row = idx / F4_ROW, c4 = idx % F4_ROW;
      if (r0 + row < S) {
        a[i] = *(const float4*)(A + (size_t)(r0 + row) * D + 4 * c4);
        b[i] = *(const float4*)(B + (size_t)(r0 + row) * D + 4 * c4);
      } else {
        a[i] = float4{0.f, 0.f, 0.f, 0.f};
        b[i] = float4{0.f, 0.f, 0.f, 0.f};
      }
    }
  }
  __device__ __forceinline__ void store(float* As, float* Bs, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = tid + kF32Waves * 64 * i;
      const int row = idx / F4_ROW, c4 = idx % F4_ROW;
      *(float4*)(As + row * KS + 4 * c4) = a[i];
      *(float4*)(Bs + row * KS + 4 * c4) = b[i];
    }
  }
};

// Transposed-accumulator store: acc[ob] rows d = 32 ob + 8 a + 4 h + 0..3,
// column = this lane's row.
template <int NOB>
__device__ __forceinline__ void store_rowT_f32(float* dst_row, const f32x16 (&acc)[NOB], int hl,
                                               float mul) {
#pragma unroll
  for (int ob = 0; ob < NOB; ++ob)
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const float4 w = {acc[ob][4 * a] * mul, acc[ob][4 * a + 1] * mul, acc[ob][4 * a + 2] * mul,
                        acc[ob][4 * a + 3] * mul};
      *(float4*)(dst_row + 32 * ob + 8 * a + 4 * hl) = w;
    }
}

// dQ: one workgroup = 128 queries of one (b, h).
template <int D, bool CAUSAL>
__global__ __launch_bounds__(kF32Waves * 64) void bwd_dq_f32_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ LD, float* __restrict__ dQ, int S,
    int Hq, int Hkv, float scale, int n_qt, int n_work) {
  constexpr int BM = 32 * kF32Waves;
  constexpr int HD = D / 2, NOB = D / 32;
  constexpr int KS = Stage2<D>::KS;
  __shared__ __attribute__((aligned(16))) float Ks[2][kF32Tile * KS];
  __shared__ __attribute__((aligned(16))) float Vs[2][kF32Tile * KS];

  const int work = xcd_remap(blockIdx.x, n_work);
  const int bh = work / n_qt;
  const int qt = n_qt - 1 - (work % n_qt);  // longest causal walks first
  const int b = bh / Hq, h = bh % Hq;
  const int hk = h / (Hq / Hkv);
  const int q0 = qt * BM;
  const size_t qoff = (size_t)(b * Hq + h) * S;
  const float* Kp = K + (size_t)(b * Hkv + hk) * S * D;
  const float* Vp = V + (size_t)(b * Hkv + hk) * S * D;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, hl = lane >> 5;
  const int qw0 = q0 + 32 * wave;
  const int myq = qw0 + l32;
  const bool qvalid = myq < S;
  const float c2 = scale * kLog2e;
  const float lse2 = qvalid ? LD[2 * (qoff + myq)] : -kNegInf;  // past S: P = 0
  const float dd = qvalid ? LD[2 * (qoff + myq) + 1] : 0.f;

  float qv[HD], gv[HD];  // Q and dO as B operands: element HD * hl + k
#pragma unroll
  for (int k4 = 0; k4 < HD; k4 += 4) {
    float4 x = {0.f, 0.f, 0.f, 0.f}, y = {0.f, 0.f, 0.f, 0.f};
    if (qvalid) {
      x = *(const float4*)(Q + (qoff + myq) * D + HD * hl + k4);
      y = *(const float4*)(dO + (qoff + myq) * D + HD * hl + k4);
    }
    qv[k4] = x.x; qv[k4 + 1] = x.y; qv[k4 + 2] = x.z; qv[k4 + 3] = x.w;
    gv[k4] = y.x; gv[k4 + 1] = y.y; gv[k4 + 2] = y.z; gv[k4 + 3] = y.w;
  }

  const int kv_end = CAUSAL ? min(S, q0 + BM) : S;
  const int n_tiles = (kv_end + kF32Tile - 1) / kF32Tile;
  Stage2<D> st;
  f32x16 acc[NOB];  // dQ^T
#pragma unroll
  for (int i = 0; i < NOB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  const int krow = krow32(l32);

  if (n_tiles > 0) st.load(Kp, Vp, 0, S, tid);
  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    st.store(Ks[buf], Vs[buf], tid);
    __syncthreads();
    if (t + 1 < n_tiles) st.load(Kp, Vp, (t + 1) * kF32Tile, S, tid);
    const int k0 = t * kF32Tile;
    if (CAUSAL && k0 > qw0 + 31) continue;  // every key after every query of the wave
    // S^T = K Q^T, dP^T = V dO^T; register r of half hl <-> key k0 + 16 hl + r
    f32x16 s, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) { s[r] = 0.f; dp[r] = 0.f; }
    const float* kr = Ks[buf] + krow * KS + HD * hl;
    const float* vr = Vs[buf] + krow * KS + HD * hl;
#pragma unroll
    for (int k4 = 0; k4 < HD; k4 += 4) {
      const float4 a = *(const float4*)(kr + k4);
      const float4 c = *(const float4*)(vr + k4);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, qv[k4], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(c.x, gv[k4], dp, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, qv[k4 + 1], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(c.y, gv[k4 + 1], dp, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, qv[k4 + 2], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(c.z, gv[k4 + 2], dp, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, qv[k4 + 3], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(c.w, gv[k4 + 3], dp, 0, 0, 0);
    }
    const bool need_mask = CAUSAL ? (k0 + kF32Tile - 1 > qw0) : (k0 + kF32Tile > S);
    float ds[16];  // dS^T / scale
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float p = fast_exp2(__builtin_fmaf(s[r], c2, -lse2));
      if (need_mask) {
        const int key = k0 + 16 * hl + r;
        if (key >= S || (CAUSAL && key > myq)) p = 0.f;
      }
      ds[r] = p * (dp[r] - dd);
    }
    // dQ^T[d x q] += K^T[d x keys] dS^T[keys x q]: step r contracts keys r, 16 + r
#pragma unroll
    for (int ob = 0; ob < NOB; ++ob) {
      const float* kt = Ks[buf] + (16 * hl) * KS + 32 * ob + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        acc[ob] = __builtin_amdgcn_mfma_f32_32x32x2f32(kt[r * KS], ds[r], acc[ob], 0, 0, 0);
    }
  }
  if (qvalid) store_rowT_f32<NOB>(dQ + (qoff + myq) * D, acc, hl, scale);
}

// dK, dV: one workgroup = 128 keys of one (b, kv head); 32-query tiles of
// every q head of the kv head.
template <int D, bool CAUSAL>
__global__ __launch_bounds__(kF32Waves * 64) void bwd_dkv_f32_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ LD, float* __restrict__ dK,
    float* __restrict__ dV, int S, int Hq, int Hkv, float scale, int n_kt, int n_work) {
  constexpr int BK = 32 * kF32Waves;
  constexpr int HD = D / 2, NOB = D / 32;
  constexpr int KS = Stage2<D>::KS;
  __shared__ __attribute__((aligned(16))) float Qs[2][kF32Tile * KS];
  __shared__ __attribute__((aligned(16))) float Gs[2][kF32Tile * KS];  // dO
  __shared__ __attribute__((aligned(16))) float Ls[2][2 * kF32Tile];   // (LSE log2 e, D) pairs

  const int work = xcd_remap(blockIdx.x, n_work);
  const int bhk = work / n_kt;
  const int kt = work % n_kt;  // causal: the first key tiles have the longest query walks
  const int b = bhk / Hkv, hk = bhk % Hkv;
  const int G = Hq / Hkv;
  const int K0 = kt * BK;
  const size_t kvoff = (size_t)(b * Hkv + hk) * S;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, hl = lane >> 5;
  const int kw0 = K0 + 32 * wave;
  const int mykey = kw0 + l32;
  const bool kvalid = mykey < S;
  const float c2 = scale * kLog2e;

  float kv[HD], vv[HD];  // K^T and V^T as B operands: element HD * hl + k of this lane's key
#pragma unroll
  for (int k4 = 0; k4 < HD; k4 += 4) {
    float4 x = {0.f, 0.f, 0.f, 0.f}, y = {0.f, 0.f, 0.f, 0.f};
    if (kvalid) {
      x = *(const float4*)(K + (kvoff + mykey) * D + HD * hl + k4);
      y = *(const float4*)(V + (kvoff + mykey) * D + HD * hl + k4);
    }
    kv[k4] = x.x; kv[k4 + 1] = x.y; kv[k4 + 2] = x.z; kv[k4 + 3] = x.w;
    vv[k4] = y.x; vv[k4 + 1] = y.y; vv[k4 + 2] = y.z; vv[k4 + 3] = y.w;
  }

  const int t_begin = CAUSAL ? K0 / kF32Tile : 0;
  const int nt = max(0, (S + kF32Tile - 1) / kF32Tile - t_begin);
  const int n_it = G * nt;
  Stage2<D> st;
  float lreg = 0.f;
  auto gload = [&](int it) {
    const int hq = hk * G + it / nt;
    const int q0 = (t_begin + it % nt) * kF32Tile;
    const size_t qoff = (size_t)(b * Hq + hq) * S;
    st.load(Q + qoff * D, dO + qoff * D, q0, S, tid);
    if (tid < 2 * kF32Tile) {  // pair element tid of the tile's 32 rows
      const int row = q0 + (tid >> 1);
      lreg = row < S ? LD[2 * (qoff + row) + (tid & 1)] : ((tid & 1) ? 0.f : -kNegInf);
    }
  };

  f32x16 dk[NOB], dv[NOB];
#pragma unroll
  for (int i = 0; i < NOB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) { dk[i][r] = 0.f; dv[i][r] = 0.f; }
  const int qrow = krow32(l32);

  if (n_it > 0) gload(0);
  for (int it = 0; it < n_it; ++it) {
    const int buf = it & 1;
    st.store(Qs[buf], Gs[buf], tid);
    if (tid < 2 * kF32Tile) Ls[buf][tid] = lreg;
    __syncthreads();
    if (it + 1 < n_it) gload(it + 1);
    const int q0 = (t_begin + it % nt) * kF32Tile;
    if (CAUSAL && q0 + 31 < kw0) continue;  // every query before every key of the wave
    // S = Q K^T, dP = dO V^T; register r of half hl <-> query q0 + 16 hl + r
    f32x16 s, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) { s[r] = 0.f; dp[r] = 0.f; }
    const float* qr = Qs[buf] + qrow * KS + HD * hl;
    const float* gr = Gs[buf] + qrow * KS + HD * hl;
#pragma unroll
    for (int k4 = 0; k4 < HD; k4 += 4) {
      const float4 a = *(const float4*)(qr + k4);
      const float4 c = *(const float4*)(gr + k4);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, kv[k4], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(c.x, vv[k4], dp, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, kv[k4 + 1], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(c.y, vv[k4 + 1], dp, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, kv[k4 + 2], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(c.z, vv[k4 + 2], dp, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, kv[k4 + 3], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(c.w, vv[k4 + 3], dp, 0, 0, 0);
    }
    const bool need_mask = !kvalid || (CAUSAL && q0 < kw0 + 31) || q0 + kF32Tile > S;
    float p[16], ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qi = 16 * hl + r;
      p[r] = fast_exp2(__builtin_fmaf(s[r], c2, -Ls[buf][2 * qi]));
      if (need_mask) {
        const int query = q0 + qi;
        if (!kvalid || query >= S || (CAUSAL && mykey > query)) p[r] = 0.f;
      }
      ds[r] = p[r] * (dp[r] - Ls[buf][2 * qi + 1]);
    }
    // dV^T[d x keys] += dO^T P, dK^T[d x keys] += Q^T dS: step r contracts
    // queries r, 16 + r
#pragma unroll
    for (int ob = 0; ob < NOB; ++ob) {
      const float* gt = Gs[buf] + (16 * hl) * KS + 32 * ob + l32;
      const float* qt = Qs[buf] + (16 * hl) * KS + 32 * ob + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        dv[ob] = __builtin_amdgcn_mfma_f32_32x32x2f32(gt[r * KS], p[r], dv[ob], 0, 0, 0);
        dk[ob] = __builtin_amdgcn_mfma_f32_32x32x2f32(qt[r * KS], ds[r], dk[ob], 0, 0, 0);
      }
    }
  }
  if (kvalid) {
    store_rowT_f32<NOB>(dK + (kvoff + mykey) * D, dk, hl, scale);
    store_rowT_f32<NOB>(dV + (kvoff + mykey) * D, dv, hl, 1.f);
  }
}

template <int D, bool CAUSAL>
hipError_t launch_bwd_f32_t(const float* q, const float* k, const float* v, const float* o,
                            const float* dout, const float* lse, float* dq, float* dk, float* dv,
                            int B, int Hq, int Hkv, int S, float scale, float* ws,
                            hipStream_t stream) {
  const long long rows = (long long)B * Hq * S;
  const long long g0 = (rows * (D / 4) + 255) / 256;
  const int n_t = (S + 32 * kF32Waves - 1) / (32 * kF32Waves);
  const long long gq = (long long)B * Hq * n_t;
  const long long gk = (long long)B * Hkv * n_t;
  if (g0 > 0x7fffffffLL || gq > 0x7fffffffLL || gk > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((bwd_rowdot_f32_kernel<D>), dim3((unsigned)g0), dim3(256), 0, stream, o, dout,
                     lse, ws, rows);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((bwd_dkv_f32_kernel<D, CAUSAL>), dim3((unsigned)gk), dim3(kF32Waves * 64), 0,
                     stream, q, k, v, dout, ws, dk, dv, S, Hq, Hkv, scale, n_t, (int)gk);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((bwd_dq_f32_kernel<D, CAUSAL>), dim3((unsigned)gq), dim3(kF32Waves * 64), 0,
                     stream, q, k, v, dout, ws, dq, S, Hq, Hkv, scale, n_t, (int)gq);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_flash_bwd_f32(const float* q, const float* k, const float* v, const float* o,
                                const float* dout, const float* lse, float* dq, float* dk,
                                float* dv, int B, int Hq, int Hkv, int S, int D, float scale,
                                bool causal, void* ws, hipStream_t stream) {
  if ((long long)B * Hq * S == 0) return hipSuccess;
  float* w = (float*)ws;
#define CA_BWD32(DD)                                                                          \
  if (D == DD)                                                                                \
    return causal ? launch_bwd_f32_t<DD, true>(q, k, v, o, dout, lse, dq, dk, dv, B, Hq, Hkv, \
                                               S, scale, w, stream)                           \
                  : launch_bwd_f32_t<DD, false>(q, k, v, o, dout, lse, dq, dk, dv, B, Hq,     \
                                                Hkv, S, scale, w, stream);
  CA_BWD32(64)
  CA_BWD32(128)
#undef CA_BWD32
  return hipErrorInvalidValue;
}

}  // namespace ca
