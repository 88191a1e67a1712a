// extern "C" entry points of include/cuda_llm_abi.h: argument validation,
// error reporting and dispatch to the gfx950 launchers.
//
// Validation mirrors the reference binding's TORCH_CHECKs
// (fused_softmax_binding.cpp:52-67 prefill, :116-132 paged, :313-322 decode,
// :650-669 fp8 paged), extended with GQA, alignment and size checks; every
// launch is followed by hipGetLastError (the reference checks nothing after
// launching, e.g. flash_attention_v2_kernel.cuh:233-304).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>
#include <algorithm>
#include <climits>
#include <initializer_list>
#include <new>
#include <vector>

#include "../../include/cuda_llm_abi.h"
#include "launch.h"

namespace {

thread_local std::string g_last_error;

ca_status fail(ca_status st, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return st;
}

ca_status from_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return CA_OK;
  if (e == hipErrorInvalidValue)
    return fail(CA_INVALID_ARGUMENT, "%s: invalid launch configuration (%s)", what,
                hipGetErrorString(e));
  return fail(CA_LAUNCH_FAILED, "%s: launch failed: %s", what, hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

ca_status check_16bit_dtype(ca_dtype dt, const char* what) {
  if (dt == CA_BF16 || dt == CA_F16) return CA_OK;
  if (dt == CA_F32)
    return fail(CA_UNSUPPORTED, "%s: float32 queries are not supported (use bf16/fp16)", what);
  return fail(CA_INVALID_ARGUMENT, "%s: unknown dtype %d", what, (int)dt);
}

// float32, fp16 or bf16: the entry points the reference instantiates for float.
ca_status check_float_dtype(ca_dtype dt, const char* what) {
  if (dt == CA_BF16 || dt == CA_F16 || dt == CA_F32) return CA_OK;
  return fail(CA_INVALID_ARGUMENT, "%s: unknown dtype %d", what, (int)dt);
}

ca_status check_heads(int hq, int hkv, const char* what) {
  if (hq <= 0 || hkv <= 0) return fail(CA_INVALID_ARGUMENT, "%s: head counts must be positive", what);
  if (hq % hkv != 0)
    return fail(CA_INVALID_ARGUMENT, "%s: num_q_heads (%d) must be a multiple of num_kv_heads (%d)",
                what, hq, hkv);
  return CA_OK;
}

ca_status check_head_dim(int d, const char* what) {
  if (d == 64 || d == 128) return CA_OK;
  return fail(CA_INVALID_ARGUMENT, "%s: Only head_dim 64 and 128 are currently supported (got %d)",
              what, d);
}

// Whether the product of non-negative factors is at most `limit`, found
// without forming a product that could overflow.
bool product_at_most(long long limit, std::initializer_list<long long> factors) {
  for (long long f : factors)
    if (f == 0) return true;
  long long p = 1;
  for (long long f : factors) {
    if (p > limit / f) return false;
    p *= f;
  }
  return true;
}

// Total elements and one (batch, head) slice: the kernels address a slice
// with 32-bit byte offsets, so its float32 size stays below 2 GiB.
ca_status check_sizes(int batch, int heads, int seq_len, int head_dim, const char* what) {
  if (!product_at_most(1LL << 40, {batch, heads, seq_len, head_dim}))
    return fail(CA_INVALID_ARGUMENT, "%s: tensor too large", what);
  if ((long long)seq_len * head_dim * 4 >= (1LL << 31))
    return fail(CA_INVALID_ARGUMENT, "%s: seq_len too long (one head's slice must stay below 2 GiB)",
                what);
  return CA_OK;
}

}  // namespace

extern "C" {

const char* ca_last_error(void) { return g_last_error.c_str(); }

const char* ca_version(void) { return "cuda_llm-amd 0.1 (gfx950)"; }

size_t ca_decode_workspace_bytes(int num_seqs, int num_q_heads, int head_dim, int max_tokens) {
  if (num_seqs <= 0 || num_q_heads <= 0 || head_dim <= 0 || max_tokens <= 0) return 0;
  return ca::decode_workspace_bytes(num_seqs, num_q_heads, head_dim, max_tokens);
}

static ca_status prefill_entry(const char* what, ca_dtype dtype, const void* q, const void* k,
                               const void* v, void* o, float* lse, int batch, int num_q_heads,
                               int num_kv_heads, int seq_len, int head_dim, float softmax_scale,
                               int is_causal, void* stream) {
  ca_status st;
  if ((st = check_float_dtype(dtype, what)) != CA_OK) return st;
  if ((st = check_heads(num_q_heads, num_kv_heads, what)) != CA_OK) return st;
  if ((st = check_head_dim(head_dim, what)) != CA_OK) return st;
  if (batch < 0 || seq_len < 0) return fail(CA_INVALID_ARGUMENT, "%s: negative size", what);
  if (batch == 0 || seq_len == 0) return CA_OK;
  if (!q || !k || !v || !o) return fail(CA_INVALID_ARGUMENT, "%s: null pointer", what);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return fail(CA_INVALID_ARGUMENT, "%s: pointers must be 16-byte aligned", what);
  if ((st = check_sizes(batch, num_q_heads, seq_len, head_dim, what)) != CA_OK) return st;
  return from_hip(ca::launch_prefill((int)dtype, q, k, v, o, lse, batch, num_q_heads,
                                     num_kv_heads, seq_len, head_dim, softmax_scale,
                                     is_causal != 0, (hipStream_t)stream),
                  what);
}

ca_status ca_flash_attention_fwd(ca_dtype dtype, const void* q, const void* k, const void* v,
                                 void* o, int batch, int num_q_heads, int num_kv_heads,
                                 int seq_len, int head_dim, float softmax_scale, int is_causal,
                                 void* stream) {
  return prefill_entry("flash_attention", dtype, q, k, v, o, nullptr, batch, num_q_heads,
                       num_kv_heads, seq_len, head_dim, softmax_scale, is_causal, stream);
}

ca_status ca_flash_attention_fwd_lse(ca_dtype dtype, const void* q, const void* k, const void* v,
                                     void* o, float* lse, int batch, int num_q_heads,
                                     int num_kv_heads, int seq_len, int head_dim,
                                     float softmax_scale, int is_causal, void* stream) {
  const char* what = "flash_attention (with lse)";
  if (!lse && batch > 0 && seq_len > 0)
    return fail(CA_INVALID_ARGUMENT, "%s: null lse pointer", what);
  return prefill_entry(what, dtype, q, k, v, o, lse, batch, num_q_heads, num_kv_heads, seq_len,
                       head_dim, softmax_scale, is_causal, stream);
}

size_t ca_flash_attention_bwd_workspace_bytes(int batch, int num_q_heads, int seq_len) {
  if (batch <= 0 || num_q_heads <= 0 || seq_len <= 0) return 0;
  return ca::bwd_workspace_bytes(batch, num_q_heads, seq_len);
}

ca_status ca_flash_attention_bwd(ca_dtype dtype, const void* q, const void* k, const void* v,
                                 const void* o, const void* dout, const float* lse, void* dq,
                                 void* dk, void* dv, int batch, int num_q_heads, int num_kv_heads,
                                 int seq_len, int head_dim, float softmax_scale, int is_causal,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  const char* what = "flash_attention_backward";
  ca_status st;
  if ((st = check_float_dtype(dtype, what)) != CA_OK) return st;
  if ((st = check_heads(num_q_heads, num_kv_heads, what)) != CA_OK) return st;
  if ((st = check_head_dim(head_dim, what)) != CA_OK) return st;
  if (batch < 0 || seq_len < 0) return fail(CA_INVALID_ARGUMENT, "%s: negative size", what);
  if (batch == 0 || seq_len == 0) return CA_OK;
  if (!q || !k || !v || !o || !dout || !lse || !dq || !dk || !dv)
    return fail(CA_INVALID_ARGUMENT, "%s: null pointer", what);
  const void* ptrs[] = {q, k, v, o, dout, dq, dk, dv};
  for (const void* p : ptrs)
    if (!aligned16(p)) return fail(CA_INVALID_ARGUMENT, "%s: pointers must be 16-byte aligned", what);
  if ((st = check_sizes(batch, num_q_heads, seq_len, head_dim, what)) != CA_OK) return st;
  const size_t need = ca::bwd_workspace_bytes(batch, num_q_heads, seq_len);
  if (workspace_bytes < need || !workspace)
    return fail(CA_INVALID_ARGUMENT, "%s: workspace of %zu bytes required, %zu given", what, need,
                workspace_bytes);
  return from_hip(ca::launch_flash_bwd((int)dtype, q, k, v, o, dout, lse, dq, dk, dv, batch,
                                       num_q_heads, num_kv_heads, seq_len, head_dim,
                                       softmax_scale, is_causal != 0, workspace,
                                       (hipStream_t)stream),
                  what);
}

ca_status ca_flash_decode(ca_dtype dtype, const void* q, const void* k, const void* v, void* o,
                          int batch, int num_q_heads, int num_kv_heads, int kv_len, int head_dim,
                          float softmax_scale, void* workspace, size_t workspace_bytes,
                          void* stream) {
  const char* what = "flash_decode";
  ca_status st;
  if ((st = check_float_dtype(dtype, what)) != CA_OK) return st;
  if ((st = check_heads(num_q_heads, num_kv_heads, what)) != CA_OK) return st;
  if ((st = check_head_dim(head_dim, what)) != CA_OK) return st;
  if (batch < 0 || kv_len < 0) return fail(CA_INVALID_ARGUMENT, "%s: negative size", what);
  if (batch == 0) return CA_OK;
  if (!q || !o || (kv_len > 0 && (!k || !v)))
    return fail(CA_INVALID_ARGUMENT, "%s: null pointer", what);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return fail(CA_INVALID_ARGUMENT, "%s: pointers must be 16-byte aligned", what);
  const size_t need = ca::decode_workspace_bytes(batch, num_q_heads, head_dim, kv_len);
  if (workspace_bytes < need || (need && !workspace))
    return fail(CA_INVALID_ARGUMENT, "%s: workspace of %zu bytes required, %zu given", what, need,
                workspace_bytes);
  return from_hip(ca::launch_flash_decode((int)dtype, q, k, v, o, batch, num_q_heads,
                                          num_kv_heads, kv_len, head_dim, softmax_scale,
                                          workspace, workspace_bytes, (hipStream_t)stream),
                  what);
}

static ca_status paged_common_checks(const char* what, const void* query, const void* kc,
                                     const void* vc, const int32_t* bt, const int32_t* lens,
                                     void* out, int num_seqs, int hq, int hkv, int head_dim,
                                     int max_blocks, int page_size, int num_blocks,
                                     void* workspace, size_t workspace_bytes,
                                     bool check_workspace = true) {
  ca_status st;
  if ((st = check_heads(hq, hkv, what)) != CA_OK) return st;
  if ((st = check_head_dim(head_dim, what)) != CA_OK) return st;
  if (page_size != 16) return fail(CA_INVALID_ARGUMENT, "%s: Only page_size 16 is currently supported (got %d)", what, page_size);
  if (num_seqs < 0 || max_blocks < 0 || num_blocks < 0)
    return fail(CA_INVALID_ARGUMENT, "%s: negative size", what);
  if (num_seqs == 0) return CA_OK;
  if (max_blocks > INT_MAX / page_size)
    return fail(CA_INVALID_ARGUMENT, "%s: block table too wide (%d entries per sequence)", what,
                max_blocks);
  if (num_blocks == 0 && max_blocks > 0)
    return fail(CA_INVALID_ARGUMENT, "%s: empty cache with a non-empty block table", what);
  if (!query || !out || !lens || (max_blocks > 0 && (!kc || !vc || !bt)))
    return fail(CA_INVALID_ARGUMENT, "%s: null pointer", what);
  if (!aligned16(query) || !aligned16(kc) || !aligned16(vc) || !aligned16(out))
    return fail(CA_INVALID_ARGUMENT, "%s: pointers must be 16-byte aligned", what);
  const size_t need = ca::decode_workspace_bytes(num_seqs, hq, head_dim, max_blocks * page_size);
  if (check_workspace && (workspace_bytes < need || (need && !workspace)))
    return fail(CA_INVALID_ARGUMENT, "%s: workspace of %zu bytes required, %zu given", what, need,
                workspace_bytes);
  return CA_OK;
}

ca_status ca_paged_attention(ca_dtype dtype, const void* query, const void* key_cache,
                             const void* value_cache, const int32_t* block_tables,
                             const int32_t* context_lens, void* out, int num_seqs,
                             int num_q_heads, int num_kv_heads, int head_dim,
                             int max_blocks_per_seq, int page_size, int num_blocks,
                             float softmax_scale, void* workspace, size_t workspace_bytes,
                             void* stream) {
  const char* what = "paged_attention";
  ca_status st;
  if ((st = check_float_dtype(dtype, what)) != CA_OK) return st;
  if ((st = paged_common_checks(what, query, key_cache, value_cache, block_tables, context_lens,
                                out, num_seqs, num_q_heads, num_kv_heads, head_dim,
                                max_blocks_per_seq, page_size, num_blocks, workspace,
                                workspace_bytes)) != CA_OK)
    return st;
  if (num_seqs == 0) return CA_OK;
  return from_hip(ca::launch_paged_decode((int)dtype, 0, query, key_cache, value_cache, nullptr,
                                          nullptr, 0, block_tables, context_lens, out, num_seqs,
                                          num_q_heads, num_kv_heads, head_dim,
                                          max_blocks_per_seq, num_blocks > 0 ? num_blocks : 1,
                                          softmax_scale, workspace, workspace_bytes,
                                          (hipStream_t)stream),
                  what);
}

ca_status ca_fp8_paged_attention(ca_dtype dtype, const void* query, const uint8_t* key_cache,
                                 const uint8_t* value_cache, const float* k_scale,
                                 const float* v_scale, int per_block_scales,
                                 const int32_t* block_tables, const int32_t* context_lens,
                                 void* out, int num_seqs, int num_q_heads, int num_kv_heads,
                                 int head_dim, int max_blocks_per_seq, int page_size,
                                 int num_blocks, float softmax_scale, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  const char* what = "fp8_paged_attention";
  ca_status st;
  if ((st = check_float_dtype(dtype, what)) != CA_OK) return st;
  if ((st = paged_common_checks(what, query, key_cache, value_cache, block_tables, context_lens,
                                out, num_seqs, num_q_heads, num_kv_heads, head_dim,
                                max_blocks_per_seq, page_size, num_blocks, workspace,
                                workspace_bytes)) != CA_OK)
    return st;
  if (num_seqs == 0) return CA_OK;
  if (!k_scale || !v_scale) return fail(CA_INVALID_ARGUMENT, "%s: null scale pointer", what);
  return from_hip(ca::launch_paged_decode((int)dtype, 1, query, key_cache, value_cache, k_scale,
                                          v_scale, per_block_scales != 0, block_tables,
                                          context_lens, out, num_seqs, num_q_heads,
                                          num_kv_heads, head_dim, max_blocks_per_seq,
                                          num_blocks > 0 ? num_blocks : 1, softmax_scale,
                                          workspace, workspace_bytes, (hipStream_t)stream),
                  what);
}

ca_status ca_fp8_paged_attention_noalloc(ca_dtype dtype, const void* query,
                                         const uint8_t* key_cache, const uint8_t* value_cache,
                                         const float* k_scale, const float* v_scale,
                                         int per_block_scales, const int32_t* block_tables,
                                         const int32_t* context_lens, void* out, int num_seqs,
                                         int num_q_heads, int num_kv_heads, int head_dim,
                                         int max_blocks_per_seq, int page_size, int num_blocks,
                                         float softmax_scale, void* stream) {
  const char* what = "fp8_paged_attention_noalloc";
  ca_status st;
  if ((st = check_float_dtype(dtype, what)) != CA_OK) return st;
  // the same checks as the workspace form, with no workspace required
  if ((st = paged_common_checks(what, query, key_cache, value_cache, block_tables, context_lens,
                                out, num_seqs, num_q_heads, num_kv_heads, head_dim,
                                max_blocks_per_seq, page_size, num_blocks, nullptr, 0,
                                false)) != CA_OK)
    return st;
  if (num_seqs == 0) return CA_OK;
  if (!k_scale || !v_scale) return fail(CA_INVALID_ARGUMENT, "%s: null scale pointer", what);
  const size_t need = ca::paged_decode_partials_bytes((int)dtype, 1, num_seqs, num_q_heads,
                                                      num_kv_heads, head_dim, max_blocks_per_seq);
  if (need > ca::kNoAllocScratchBytes)
    return fail(CA_INVALID_ARGUMENT,
                "%s: these sizes need %zu bytes of split partials, more than the %zu bytes of "
                "the library's scratch (use ca_fp8_paged_attention with a workspace)",
                what, need, ca::kNoAllocScratchBytes);
  auto launch = [&](void* scratch) {
    return ca::launch_paged_decode((int)dtype, 1, query, key_cache, value_cache, k_scale, v_scale,
                                   per_block_scales != 0, block_tables, context_lens, out, num_seqs,
                                   num_q_heads, num_kv_heads, head_dim, max_blocks_per_seq,
                                   num_blocks > 0 ? num_blocks : 1, softmax_scale, scratch, need,
                                   (hipStream_t)stream);
  };
  // one split needs no partials; otherwise the scratch, serialised per device
  if (need == 0) return from_hip(launch(nullptr), what);
  return from_hip(ca::with_noalloc_scratch((hipStream_t)stream, launch), what);
}

size_t ca_mx_workspace_bytes(ca_scale_kind scale_kind, int batch, int num_heads, int seq_len,
                             int head_dim) {
  if (batch <= 0 || num_heads <= 0 || seq_len <= 0 || head_dim != 128) return 0;
  if (scale_kind != CA_SCALE_E8M0 && scale_kind != CA_SCALE_F32) return 0;
  return ca::mx_workspace_bytes((int)scale_kind, batch, num_heads, seq_len, head_dim);
}

ca_status ca_fused_microscaled_attention(ca_dtype out_dtype, const uint8_t* q, const void* q_scale,
                                         const uint8_t* k, const void* k_scale, const uint8_t* v,
                                         const void* v_scale, ca_scale_kind scale_kind, void* out,
                                         int batch, int num_heads, int seq_len, int head_dim,
                                         float softmax_scale, int is_causal, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  const char* what = "fused_microscaled_attention";
  if (out_dtype != CA_BF16 && out_dtype != CA_F16)
    return fail(out_dtype == CA_F32 ? CA_UNSUPPORTED : CA_INVALID_ARGUMENT,
                "%s: output dtype must be bf16 or fp16", what);
  if (scale_kind != CA_SCALE_E8M0 && scale_kind != CA_SCALE_F32)
    return fail(CA_INVALID_ARGUMENT, "%s: unknown scale kind %d", what, (int)scale_kind);
  if (head_dim != 128)
    return fail(CA_INVALID_ARGUMENT, "%s: head_dim must be 128 (got %d)", what, head_dim);
  if (batch < 0 || num_heads < 0 || seq_len < 0)
    return fail(CA_INVALID_ARGUMENT, "%s: negative size", what);
  if (batch == 0 || num_heads == 0 || seq_len == 0) return CA_OK;
  if (!q || !k || !v || !q_scale || !k_scale || !v_scale || !out)
    return fail(CA_INVALID_ARGUMENT, "%s: null pointer", what);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || !aligned16(workspace))
    return fail(CA_INVALID_ARGUMENT, "%s: code/output/workspace pointers must be 16-byte aligned",
                what);
  const uintptr_t scale_align = scale_kind == CA_SCALE_F32 ? 4u : 1u;
  if ((reinterpret_cast<uintptr_t>(q_scale) | reinterpret_cast<uintptr_t>(v_scale)) & (scale_align - 1))
    return fail(CA_INVALID_ARGUMENT, "%s: float scales must be 4-byte aligned", what);
  if (((reinterpret_cast<uintptr_t>(q_scale) | reinterpret_cast<uintptr_t>(k_scale)) & 3u) != 0)
    return fail(CA_INVALID_ARGUMENT, "%s: q_scale and k_scale must be 4-byte aligned", what);
  ca_status st;
  if ((st = check_sizes(batch, num_heads, seq_len, head_dim, what)) != CA_OK) return st;
  const size_t need = ca::mx_workspace_bytes((int)scale_kind, batch, num_heads, seq_len, head_dim);
  if (workspace_bytes < need || !workspace)
    return fail(CA_INVALID_ARGUMENT, "%s: workspace of %zu bytes required, %zu given", what, need,
                workspace_bytes);
  return from_hip(
      ca::launch_mxfp8((int)out_dtype, (int)scale_kind, q, q_scale, k, k_scale, v, v_scale, out,
                       batch, num_heads, seq_len, head_dim, softmax_scale, is_causal != 0, workspace,
                       workspace_bytes, (hipStream_t)stream),
      what);
}

ca_status ca_check_mx_scales(const float* q_scale, const float* k_scale, const float* v_scale,
                             int batch, int num_heads, int seq_len, int head_dim, void* stream) {
  const char* what = "check_mx_scales";
  if (batch < 0 || num_heads < 0 || seq_len < 0 || head_dim <= 0 || head_dim % 32)
    return fail(CA_INVALID_ARGUMENT, "%s: negative size or head_dim not a multiple of 32", what);
  const long long n = (long long)batch * num_heads * seq_len * (head_dim / 32);
  if (n == 0) return CA_OK;
  if (!q_scale || !k_scale || !v_scale) return fail(CA_INVALID_ARGUMENT, "%s: null pointer", what);
  if ((reinterpret_cast<uintptr_t>(q_scale) | reinterpret_cast<uintptr_t>(k_scale) |
       reinterpret_cast<uintptr_t>(v_scale)) & 3u)
    return fail(CA_INVALID_ARGUMENT, "%s: float scales must be 4-byte aligned", what);
  bool bad = false;
  ca_status st = from_hip(ca::check_mx_scales(q_scale, k_scale, v_scale, n, &bad, (hipStream_t)stream), what);
  if (st != CA_OK) return st;
  if (bad)
    return fail(CA_INVALID_ARGUMENT,
                "%s: float MX scales must be powers of two in [2^-127, 2^127] (the e8m0 values)",
                what);
  return CA_OK;
}

size_t ca_rope_workspace_bytes(ca_dtype dtype, int batch, int num_q_heads, int num_kv_heads,
                               int seq_len, int head_dim) {
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || seq_len <= 0 || head_dim <= 0)
    return 0;
  return ca::rope_workspace_bytes((int)dtype, batch, num_q_heads, num_kv_heads, seq_len,
                                  head_dim);
}

ca_status ca_fused_rope_flash_attention(ca_dtype dtype, const void* q, const void* k,
                                        const void* v, const float* cos_tab, const float* sin_tab,
                                        void* o, int batch, int num_q_heads, int num_kv_heads,
                                        int seq_len, int head_dim, float softmax_scale,
                                        int is_causal, void* workspace, size_t workspace_bytes,
                                        void* stream) {
  const char* what = "fused_rope_flash_attention";
  ca_status st;
  if ((st = check_float_dtype(dtype, what)) != CA_OK) return st;
  if ((st = check_heads(num_q_heads, num_kv_heads, what)) != CA_OK) return st;
  if ((st = check_head_dim(head_dim, what)) != CA_OK) return st;
  if (batch < 0 || seq_len < 0) return fail(CA_INVALID_ARGUMENT, "%s: negative size", what);
  if (batch == 0 || seq_len == 0) return CA_OK;
  if (!q || !k || !v || !o || !cos_tab || !sin_tab)
    return fail(CA_INVALID_ARGUMENT, "%s: null pointer", what);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || !aligned16(workspace) ||
      !aligned16(cos_tab) || !aligned16(sin_tab))
    return fail(CA_INVALID_ARGUMENT, "%s: pointers must be 16-byte aligned", what);
  if ((st = check_sizes(batch, num_q_heads, seq_len, head_dim, what)) != CA_OK) return st;
  const size_t need = ca::rope_workspace_bytes((int)dtype, batch, num_q_heads, num_kv_heads,
                                               seq_len, head_dim);
  if (workspace_bytes < need || !workspace)
    return fail(CA_INVALID_ARGUMENT, "%s: workspace of %zu bytes required, %zu given", what, need,
                workspace_bytes);
  return from_hip(ca::launch_rope_prefill((int)dtype, q, k, v, cos_tab, sin_tab, o, batch,
                                          num_q_heads, num_kv_heads, seq_len, head_dim,
                                          softmax_scale, is_causal != 0, workspace,
                                          (hipStream_t)stream),
                  what);
}

ca_status ca_check_block_tables(const int32_t* block_tables, const int32_t* context_lens,
                                int num_seqs, int max_blocks_per_seq, int num_blocks,
                                int page_size, void* stream) {
  const char* what = "check_block_tables";
  if (num_seqs < 0 || max_blocks_per_seq < 0 || num_blocks < 0 || page_size <= 0)
    return fail(CA_INVALID_ARGUMENT, "%s: negative size or page size", what);
  if (num_seqs == 0) return CA_OK;
  if (!context_lens || (max_blocks_per_seq > 0 && !block_tables))
    return fail(CA_INVALID_ARGUMENT, "%s: null pointer", what);
  // the tables may still be being written on `stream`
  hipError_t e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) return fail(CA_LAUNCH_FAILED, "%s: %s", what, hipGetErrorString(e));
  // host memory stays bounded: lengths and table entries go through buffers
  // of at most kChunk entries, runs of whole rows at a time (a row longer
  // than kChunk in pieces)
  constexpr size_t kChunk = size_t(1) << 20;
  const size_t W = (size_t)max_blocks_per_seq;
  const int rows = (int)std::min<size_t>({(size_t)num_seqs, kChunk, W ? std::max<size_t>(1, kChunk / W) : kChunk});
  try {
    std::vector<int32_t> lens((size_t)rows), buf(std::min(W * rows, kChunk));
    for (int n0 = 0; n0 < num_seqs; n0 += rows) {
      const int nr = std::min(rows, num_seqs - n0);
      e = hipMemcpy(lens.data(), context_lens + n0, (size_t)nr * sizeof(int32_t), hipMemcpyDeviceToHost);
      const bool whole = W * nr <= kChunk;   // the run's rows in one copy
      if (e == hipSuccess && whole && W)
        e = hipMemcpy(buf.data(), block_tables + (size_t)n0 * W, W * nr * sizeof(int32_t), hipMemcpyDeviceToHost);
      if (e != hipSuccess) return fail(CA_LAUNCH_FAILED, "%s: copy failed: %s", what, hipGetErrorString(e));
      for (int i = 0; i < nr; ++i) {
        const int n = n0 + i;
        const long long len = lens[(size_t)i] < 0 ? 0 : lens[(size_t)i];
        const long long used = std::min<long long>((len + page_size - 1) / page_size, max_blocks_per_seq);
        for (long long j0 = 0; j0 < used; j0 += (long long)buf.size()) {
          const long long m = std::min<long long>((long long)buf.size(), used - j0);
          const int32_t* row = buf.data() + (whole ? (size_t)i * W : 0);
          if (!whole) {
            e = hipMemcpy(buf.data(), block_tables + (size_t)n * W + j0, (size_t)m * sizeof(int32_t),
                          hipMemcpyDeviceToHost);
            if (e != hipSuccess)
              return fail(CA_LAUNCH_FAILED, "%s: copy failed: %s", what, hipGetErrorString(e));
          }
          for (long long j = 0; j < m; ++j) {
            const int32_t id = row[whole ? j0 + j : j];
            if (id < 0 || id >= num_blocks)
              return fail(CA_INVALID_ARGUMENT,
                          "%s: block_tables[%d][%lld] = %d is outside the pool [0, %d) (context length %lld)",
                          what, n, j0 + j, (int)id, num_blocks, len);
          }
          if (whole) break;   // the whole row is in buf
        }
      }
    }
  } catch (const std::bad_alloc&) {
    return fail(CA_LAUNCH_FAILED, "%s: out of host memory", what);
  }
  return CA_OK;
}

ca_status ca_stream_read(const void* p, size_t bytes, void* sink, void* stream) {
  const char* what = "stream_read";
  if (bytes == 0) return CA_OK;
  if (!p || !sink) return fail(CA_INVALID_ARGUMENT, "%s: null pointer", what);
  if (!aligned16(p) || bytes % 16)
    return fail(CA_INVALID_ARGUMENT, "%s: pointer and size must be 16-byte aligned", what);
  return from_hip(ca::launch_stream_read(p, bytes, sink, (hipStream_t)stream), what);
}

ca_status ca_paged_kv_append(ca_dtype dtype, int cache_kind, const void* key, const void* value,
                             void* key_cache, void* value_cache, float* k_scale, float* v_scale,
                             int per_block_scales, const int32_t* block_tables,
                             const int32_t* context_lens, const int32_t* new_lens, int num_seqs,
                             int num_kv_heads, int head_dim, int max_new_tokens,
                             int max_blocks_per_seq, int num_blocks, void* stream) {
  const char* what = "paged_kv_append";
  ca_status st;
  if ((st = check_16bit_dtype(dtype, what)) != CA_OK) return st;
  if ((st = check_head_dim(head_dim, what)) != CA_OK) return st;
  if (cache_kind != 0 && cache_kind != 1)
    return fail(CA_INVALID_ARGUMENT, "%s: unknown cache kind %d", what, cache_kind);
  if (num_kv_heads <= 0) return fail(CA_INVALID_ARGUMENT, "%s: num_kv_heads must be positive", what);
  if (num_seqs < 0 || max_new_tokens < 0 || max_blocks_per_seq < 0 || num_blocks < 0)
    return fail(CA_INVALID_ARGUMENT, "%s: negative size", what);
  if (num_seqs == 0 || max_new_tokens == 0 || max_blocks_per_seq == 0) return CA_OK;
  if (!key || !value || !key_cache || !value_cache || !block_tables || !context_lens)
    return fail(CA_INVALID_ARGUMENT, "%s: null pointer", what);
  if (!aligned16(key_cache) || !aligned16(value_cache))
    return fail(CA_INVALID_ARGUMENT, "%s: caches must be 16-byte aligned", what);
  if (cache_kind == 1 && (!k_scale || !v_scale))
    return fail(CA_INVALID_ARGUMENT, "%s: FP8 caches need k_scale and v_scale", what);
  if (!product_at_most(1LL << 40, {num_seqs, num_kv_heads, max_new_tokens, head_dim}))
    return fail(CA_INVALID_ARGUMENT, "%s: tensor too large", what);
  const int kind = cache_kind == 0 ? 0 : (per_block_scales ? 2 : 1);
  return from_hip(ca::launch_kv_append((int)dtype, kind, key, value, key_cache, value_cache,
                                       k_scale, v_scale, block_tables, context_lens, new_lens,
                                       num_seqs, num_kv_heads, head_dim, max_new_tokens,
                                       max_blocks_per_seq, num_blocks, (hipStream_t)stream),
                  what);
}

}  // extern "C"
