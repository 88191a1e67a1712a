// Internal launcher declarations shared by the kernel translation units and
// the C ABI (abi.cpp). Not part of the public interface.
#pragma once

#include <hip/hip_runtime.h>

#include <functional>
#include <stddef.h>
#include <stdint.h>

#include <atomic>

namespace ca {

// dtype codes; the same values as ca_dtype in include/cuda_llm_abi.h
constexpr int kDtypeF32 = 0;
constexpr int kDtypeF16 = 1;
constexpr int kDtypeBF16 = 2;

// RoPE tables (fp32 [S, D], rotate-half) applied to Q as the 16-bit prefill
// kernels load it; null: no rotation.
struct RopeQ {
  const float* cos = nullptr;
  const float* sin = nullptr;
};

// Prefill; lse (may be null) receives the natural-log row logsumexp [B, Hq, S].
// rq (16-bit dtypes only) rotates q on load.
hipError_t launch_prefill(int dtype, const void* q, const void* k, const void* v, void* o,
                          float* lse, int B, int Hq, int Hkv, int S, int D, float scale,
                          bool causal, hipStream_t stream, RopeQ rq = RopeQ{});
// 64-row-per-wave prefill (prefill_w64.hip): bf16 or fp16 (f16), head dim
// 128, softmax scale >= 0, no RoPE; launch_prefill dispatches to it when
// supported.
bool prefill_w64_supported(int D, int S, float scale, bool rope);
hipError_t launch_prefill_w64(bool f16, const void* q, const void* k, const void* v, void* o, float* lse, int B,
                              int Hq, int Hkv, int S, float scale, bool causal, hipStream_t stream);
void magic_div(uint32_t d, uint32_t* m, uint32_t* sh);
// Work decomposition of the 64-row kernels (grid 0: nothing to launch).
struct PfW64Geom {
  long long grid;
  int n_qt, n_work, paired, q_shift, n_bh, n_full, half;
  uint32_t m_nqt, sh_nqt, m_half, sh_half;
  int xcd_q, xcd_r;
};
hipError_t w64_geometry(int B, int Hq, int S, bool causal, PfW64Geom* g);
// The MXFP8 form (prefill_w64_mx.hip): e4m3 Q, K with e8m0 scales [rows][4],
// bf16 V, bf16 (out_f16 false) or fp16 output; any finite softmax scale,
// S < 2^22 and B * H * S < 2^30 (else hipErrorInvalidValue).
hipError_t launch_prefill_w64_mx(bool out_f16, const uint8_t* q, const uint8_t* qs, const uint8_t* k,
                                 const uint8_t* ks, const uint16_t* v_bf16, void* o, int B, int H, int S,
                                 float scale, bool causal, hipStream_t stream);

// float32 prefill (f32.hip)
hipError_t launch_prefill_f32(const void* q, const void* k, const void* v, void* o, float* lse,
                              int B, int Hq, int Hkv, int S, int D, float scale, bool causal,
                              hipStream_t stream);

// Backward (backward.hip): dq, dk, dv from q, k, v, o, dout and the forward's
// natural-log LSE; ws holds bwd_workspace_bytes (per query row the pair
// (LSE * log2(e), rowsum(dO * O))).
size_t bwd_workspace_bytes(int B, int Hq, int S);
hipError_t launch_flash_bwd(int dtype, const void* q, const void* k, const void* v,
                            const void* o, const void* dout, const float* lse, void* dq, void* dk,
                            void* dv, int B, int Hq, int Hkv, int S, int D, float scale,
                            bool causal, void* ws, hipStream_t stream);

// float32 backward (backward_f32.hip), same contract and workspace
hipError_t launch_flash_bwd_f32(const float* q, const float* k, const float* v, const float* o,
                                const float* dout, const float* lse, float* dq, float* dk,
                                float* dv, int B, int Hq, int Hkv, int S, int D, float scale,
                                bool causal, void* ws, hipStream_t stream);

// Compute units of the current device (cached per device; 0 if unknown).
// Safe for concurrent first calls: each slot is an atomic, and every thread
// that finds it empty stores the same attribute value.
inline int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Workgroups of a prefill launch of n_qt query tiles per (b, h). A causal
// launch pairs query tiles (prefill_work: n_qt-1-p with p of a head, the
// middle tiles of an odd n_qt two heads at a time) when the paired grid still
// gives every workgroup slot of the device at least one workgroup; otherwise
// each workgroup takes one tile.
inline long long prefill_grid(int B, int Hq, int n_qt, bool causal, int wg_per_cu, int* paired) {
  const long long n_bh = (long long)B * Hq;
  const long long single = n_bh * n_qt;
  const long long pairs = n_bh * (n_qt / 2) + ((n_qt & 1) ? (n_bh + 1) / 2 : 0);
  *paired = (causal && n_qt > 1 && pairs >= (long long)device_cus() * wg_per_cu) ? 1 : 0;
  return *paired ? pairs : single;
}

// Split-K geometry of the decode kernels: pages of 16 tokens. The
// workspace and the contiguous-cache kernel split at kPagesPerWave pages
// (one page id per lane of a wave); the paged kernels split at a multiple of
// it (decode.hip, DmaCfg), so the workspace sized for kPagesPerWave-page
// splits covers them.
constexpr int kDecodePage = 16;
constexpr int kPagesPerWave = 64;
constexpr int kDecodeWgWaves = 4;  // independent waves per workgroup (contiguous kernel)

// Workspace for split-K partial results: [N][Hq][max_splits] x (D + 1) floats.
size_t decode_workspace_bytes(int N, int Hq, int D, int max_tokens);

// Paged decode. cache_kind: 0 = 16-bit cache of the query dtype, 1 = fp8 e4m3
// bytes with fp32 scales (per head [Hkv] or per block [num_blocks, Hkv]).
hipError_t launch_paged_decode(int dtype, int cache_kind, const void* q, const void* kc,
                               const void* vc, const float* k_scale, const float* v_scale,
                               int per_block_scales, const int32_t* block_tables,
                               const int32_t* context_lens, void* out, int N, int Hq, int Hkv,
                               int D, int max_blocks_per_seq, int num_blocks, float scale,
                               void* ws, size_t ws_bytes, hipStream_t stream);

// Bytes of partials a paged decode launch writes on the current device (the
// exact minimum of its workspace; the entry points require
// decode_workspace_bytes, which is at least this).
size_t paged_decode_partials_bytes(int dtype, int cache_kind, int N, int Hq, int Hkv, int D,
                                   int max_blocks_per_seq);

// The allocation-free paged decode's scratch (decode.hip): a file-scope
// device array of kNoAllocScratchBytes per device; *ptr receives its address
// on the current device (looked up once per device).
constexpr size_t kNoAllocScratchBytes = 16u << 20;
// Runs `run` with the device address of this device's allocation-free
// scratch, serialised against the previous call on the device (see decode.hip).
hipError_t with_noalloc_scratch(hipStream_t stream, const std::function<hipError_t(void*)>& run);

// Contiguous-cache decode (q_len = 1 over k/v [B, Hkv, S, D]).
hipError_t launch_flash_decode(int dtype, const void* q, const void* k, const void* v, void* o,
                               int B, int Hq, int Hkv, int S, int D, float scale, void* ws,
                               size_t ws_bytes, hipStream_t stream);

// Paged KV-cache append (kv_append.hip). kind: 0 = 16-bit cache of the key
// dtype, 1 = fp8 e4m3 with per-head scales [Hkv], 2 = fp8 e4m3 with per-page
// scales [num_blocks, Hkv] (re-quantised over every touched page).
hipError_t launch_kv_append(int dtype, int kind, const void* key, const void* value, void* kc,
                            void* vc, float* k_scale, float* v_scale, const int32_t* block_tables,
                            const int32_t* context_lens, const int32_t* new_lens, int N, int Hkv,
                            int D, int T, int max_blocks, int num_blocks, hipStream_t stream);

// RoPE + prefill (rope.hip): q and k rotated into ws, then launch_prefill.
size_t rope_workspace_bytes(int dtype, int B, int Hq, int Hkv, int S, int D);
hipError_t launch_rope_prefill(int dtype, const void* q, const void* k, const void* v,
                               const float* cos_tab, const float* sin_tab, void* o, int B, int Hq,
                               int Hkv, int S, int D, float scale, bool causal, void* ws,
                               hipStream_t stream);

// Streaming read of `bytes` (multiple of 16) for the bandwidth ceiling (stream_read.hip).
hipError_t launch_stream_read(const void* p, size_t bytes, void* sink, hipStream_t stream);

// MXFP8 attention (mxfp8.hip): e4m3 q/k/v [B, H, S, D] with scales [B, H, S,
// D/32], e8m0 bytes (scale_kind 0) or float32 powers of two (scale_kind 1);
// ws holds mx_workspace_bytes (V dequantised to bf16; with float scales the
// converted q/k scale bytes). Asynchronous in both forms: a float scale that
// is not a power of two in [2^-127, 2^127] becomes the e8m0 NaN, so the
// outputs it reaches are not meaningful; check_mx_scales reports such scales.
size_t mx_workspace_bytes(int scale_kind, int B, int H, int S, int D);
hipError_t launch_mxfp8(int out_dtype, int scale_kind, const uint8_t* q, const void* qs,
                        const uint8_t* k, const void* ks, const uint8_t* v, const void* vs, void* o,
                        int B, int H, int S, int D, float scale, bool causal, void* ws,
                        size_t ws_bytes, hipStream_t stream);
// Synchronous: waits for `stream`, then sets *bad if any of the n entries of
// the three float scale arrays is not a power of two in [2^-127, 2^127].
hipError_t check_mx_scales(const float* qs, const float* ks, const float* vs, long long n, bool* bad,
                           hipStream_t stream);

}  // namespace ca
