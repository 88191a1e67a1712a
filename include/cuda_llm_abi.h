/*
 * cuda_llm_abi.h — C ABI of the MI355X (gfx950) attention forward hot path.
 *
 * Drop-in boundary for the reference's host API (kernels_api.h). The
 * reference exposes C++ templates instantiated per element type; this ABI
 * takes the element type as an enum argument and returns a status code, so
 * any FFI (ctypes, cffi, a torch extension, another language) can bind it.
 *
 * Conventions
 *  - All tensor arguments are raw device pointers to contiguous row-major
 *    buffers in the layouts stated per function; 16-byte aligned.
 *  - The library never allocates, frees or retains caller memory. Decode
 *    (split-K or the balanced walk of larger paged launches, whose partial
 *    results are merged) needs a caller-provided workspace of
 *    ca_decode_workspace_bytes()
 *    (ca_fp8_paged_attention_noalloc instead uses a fixed scratch array the
 *    library holds per device).
 *  - `stream` is a hipStream_t (NULL = the default stream). Calls enqueue
 *    work asynchronously and never synchronise the host.
 *  - Non-OK status: ca_last_error() returns a thread-local message.
 *  - Element types: CA_BF16 and CA_F16 for 16-bit q/k/v/out everywhere;
 *    CA_F32 for prefill (with and without LSE), backward, RoPE prefill,
 *    flash_decode, paged and FP8 paged decode (the entry points the reference
 *    instantiates for float). paged_kv_append takes CA_BF16 / CA_F16 only, and
 *    MXFP8 writes CA_BF16 / CA_F16 outputs.
 *  - head_dim must be 64 or 128 (fused_softmax_binding.cpp:65-67); the MXFP8
 *    entry point requires 128.
 *  - GQA: num_q_heads % num_kv_heads == 0, kv head = q head / (Hq / Hkv)
 *    (fused_gqa_kernel.cuh:40-41, tests/_utils.py:67-72).
 */
#ifndef CUDA_LLM_ABI_H
#define CUDA_LLM_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The enums are int-sized in C and C++; in C++ they have int as their fixed
 * underlying type, so any int a caller passes (an unknown dtype from a
 * binding, say) is a valid value that the checks reject, not undefined
 * behaviour. */
#ifdef __cplusplus
#define CA_ENUM_INT : int
#else
#define CA_ENUM_INT
#endif

typedef enum CA_ENUM_INT {
  CA_OK = 0,
  CA_INVALID_ARGUMENT = 1,
  CA_UNSUPPORTED = 2,
  CA_LAUNCH_FAILED = 3
} ca_status;

typedef enum CA_ENUM_INT { CA_F32 = 0, CA_F16 = 1, CA_BF16 = 2 } ca_dtype;

/* Prefill forward: O = softmax(Q K^T * scale [+ causal mask]) V.
 * q, o: [batch, num_q_heads, seq_len, head_dim]; k, v: [batch, num_kv_heads,
 * seq_len, head_dim]. Causal masking is top-left aligned (key j visible to
 * query i iff j <= i).
 * Replaces dispatch_flash_attention_v2<T> (kernels_api.h:29-33),
 * dispatch_flash_attention_v3_hopper<T> (kernels_api.h:78-83) and
 * dispatch_fused_gqa<T> (kernels_api.h:52-56). */
ca_status ca_flash_attention_fwd(ca_dtype dtype, const void* q, const void* k, const void* v,
                                 void* o, int batch, int num_q_heads, int num_kv_heads,
                                 int seq_len, int head_dim, float softmax_scale, int is_causal,
                                 void* stream);

/* Prefill forward that also writes the natural-log row logsumexp of the
 * scaled, masked scores, lse: [batch, num_q_heads, seq_len] float32 (-inf for
 * a row with no visible key). No counterpart in the reference: its forward
 * returns O only, while its backward consumes this LSE
 * (flash_attention_bwd_kernel.cuh:31, fused_softmax_binding.cpp:367-376;
 * the reference tests build it with ref_lse, tests/_utils.py:56-64). Same
 * arguments and checks as ca_flash_attention_fwd. */
ca_status ca_flash_attention_fwd_lse(ca_dtype dtype, const void* q, const void* k, const void* v,
                                     void* o, float* lse, int batch, int num_q_heads,
                                     int num_kv_heads, int seq_len, int head_dim,
                                     float softmax_scale, int is_causal, void* stream);

/* Backward of the prefill forward: dq, dk, dv from q, k, v, the forward output
 * o, its gradient dout and the forward's natural-log LSE [batch, num_q_heads,
 * seq_len] float32. q, o, dout, dq: [batch, num_q_heads, seq_len, head_dim];
 * k, v, dk, dv: [batch, num_kv_heads, seq_len, head_dim] (GQA: dk, dv sum
 * over the q heads of a kv head). dtype float32, fp16 or bf16.
 * Replaces dispatch_flash_attention_v2_backward<T> (kernels_api.h:65-69);
 * dq, dk, dv are written, not accumulated. workspace:
 * ca_flash_attention_bwd_workspace_bytes(batch, num_q_heads, seq_len). */
ca_status ca_flash_attention_bwd(ca_dtype dtype, const void* q, const void* k, const void* v,
                                 const void* o, const void* dout, const float* lse, void* dq,
                                 void* dk, void* dv, int batch, int num_q_heads, int num_kv_heads,
                                 int seq_len, int head_dim, float softmax_scale, int is_causal,
                                 void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of the ca_flash_attention_bwd workspace: per query row the pair
 * (lse * log2(e), rowsum(dout * o)), 8 bytes. */
size_t ca_flash_attention_bwd_workspace_bytes(int batch, int num_q_heads, int seq_len);

/* Prefill forward on RoPE-rotated q and k (rotate-half convention):
 * x'[c] = x[c] cos[s][c] + r[c] sin[s][c], r = [-x[D/2:], x[:D/2]], for the
 * token at position s; cos_tab, sin_tab: float32 [seq_len, head_dim]. Shapes,
 * masking and dtypes as ca_flash_attention_fwd (GQA allowed).
 * Replaces dispatch_fused_rope_flash_attention<T> (kernels_api.h:44-49).
 * workspace: ca_rope_workspace_bytes(...) (the rotated k; for float32 the
 * rotated q as well: the 16-bit kernels rotate q as they load it). */
ca_status ca_fused_rope_flash_attention(ca_dtype dtype, const void* q, const void* k,
                                        const void* v, const float* cos_tab, const float* sin_tab,
                                        void* o, int batch, int num_q_heads, int num_kv_heads,
                                        int seq_len, int head_dim, float softmax_scale,
                                        int is_causal, void* workspace, size_t workspace_bytes,
                                        void* stream);

/* Bytes of the ca_fused_rope_flash_attention workspace. */
size_t ca_rope_workspace_bytes(ca_dtype dtype, int batch, int num_q_heads, int num_kv_heads,
                               int seq_len, int head_dim);

/* Measurement helper, no counterpart in the reference: reads `bytes` bytes
 * (a multiple of 16, 16-byte aligned) from device memory at `p` with
 * streaming loads; `sink` is a 4-byte device word the kernel may write. The
 * time of this call is the measured streaming-read ceiling that the
 * HBM-bound decode entry points are compared with. */
ca_status ca_stream_read(const void* p, size_t bytes, void* sink, void* stream);

/* Append new tokens to a paged KV cache, in place: the step before paged
 * decode. key, value: [num_seqs, num_kv_heads, max_new_tokens, head_dim] of
 * `dtype` (bf16/fp16); sequence n appends its first new_lens[n] tokens
 * (new_lens NULL: max_new_tokens each) at positions context_lens[n] ..
 * through block_tables [num_seqs, max_blocks_per_seq]: the token at position
 * t goes to cache[block_tables[n][t / 16]][h][:, t % 16], the layout of the
 * paged decode entry points (tests/_utils.py:105-133).
 *   cache_kind 0: 16-bit caches of `dtype`;
 *   cache_kind 1: e4m3 code caches (uint8) with float32 scales, per head
 *     [num_kv_heads] (new slots: e4m3(x / scale), saturated) or, with
 *     per_block_scales, per (page, kv head) [num_blocks, num_kv_heads]: each
 *     touched page is quantised again over its valid slots with scale =
 *     max(amax / 448, 1e-8) (the reference's recipe, tests/
 *     test_kernels_misc.py:52-55, per page), and its scale is written.
 * Positions past the table and block ids outside [0, num_blocks) are skipped.
 * No counterpart in the reference (it builds caches in torch); the format is
 * the one ca_paged_attention and ca_fp8_paged_attention read. context_lens is
 * not updated. */
ca_status ca_paged_kv_append(ca_dtype dtype, int cache_kind, const void* key, const void* value,
                             void* key_cache, void* value_cache, float* k_scale, float* v_scale,
                             int per_block_scales, const int32_t* block_tables,
                             const int32_t* context_lens, const int32_t* new_lens, int num_seqs,
                             int num_kv_heads, int head_dim, int max_new_tokens,
                             int max_blocks_per_seq, int num_blocks, void* stream);

/* Single-token decode over a contiguous cache.
 * q, o: [batch, num_q_heads, 1, head_dim]; k, v: [batch, num_kv_heads, kv_len,
 * head_dim]. Replaces dispatch_async_flash_decode<T> (kernels_api.h:58-62).
 * workspace: ca_decode_workspace_bytes(batch, num_q_heads, head_dim, kv_len). */
ca_status ca_flash_decode(ca_dtype dtype, const void* q, const void* k, const void* v, void* o,
                          int batch, int num_q_heads, int num_kv_heads, int kv_len, int head_dim,
                          float softmax_scale, void* workspace, size_t workspace_bytes,
                          void* stream);

/* Paged decode (vLLM layout), 16-bit cache of the query dtype.
 * query, out: [num_seqs, num_q_heads, head_dim]; key_cache, value_cache:
 * [num_blocks, num_kv_heads, head_dim, page_size] (page axis innermost);
 * block_tables: int32 [num_seqs, max_blocks_per_seq]; context_lens: int32
 * [num_seqs]. page_size must be 16. A sequence with context_len <= 0 gets a
 * zero output row. Block ids outside [0, num_blocks) are clamped
 * (ca_check_block_tables reports them).
 * Replaces dispatch_paged_attention<T> (kernels_api.h:35-41).
 * workspace: ca_decode_workspace_bytes(num_seqs, num_q_heads, head_dim,
 * max_blocks_per_seq * page_size). */
ca_status ca_paged_attention(ca_dtype dtype, const void* query, const void* key_cache,
                             const void* value_cache, const int32_t* block_tables,
                             const int32_t* context_lens, void* out, int num_seqs,
                             int num_q_heads, int num_kv_heads, int head_dim,
                             int max_blocks_per_seq, int page_size, int num_blocks,
                             float softmax_scale, void* workspace, size_t workspace_bytes,
                             void* stream);

/* FP8 paged decode: caches hold OCP e4m3 codes (1 byte each) in the paged
 * layout above; k = code * k_scale, v = code * v_scale with fp32 scales per
 * kv head ([num_kv_heads], per_block_scales = 0) or per (physical block, kv
 * head) ([num_blocks, num_kv_heads], per_block_scales = 1). Output in the
 * query dtype. Replaces dispatch_fp8_paged_attention<T_OUT, T_Q>
 * (kernels_api.h:94-101), whose kernel decodes int8 rather than e4m3
 * (fp8_paged_attention_kernel.cuh:102,135). */
ca_status ca_fp8_paged_attention(ca_dtype dtype, const void* query, const uint8_t* key_cache,
                                 const uint8_t* value_cache, const float* k_scale,
                                 const float* v_scale, int per_block_scales,
                                 const int32_t* block_tables, const int32_t* context_lens,
                                 void* out, int num_seqs, int num_q_heads, int num_kv_heads,
                                 int head_dim, int max_blocks_per_seq, int page_size,
                                 int num_blocks, float softmax_scale, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* FP8 paged decode that allocates nothing and takes no workspace: the
 * arguments, checks and results of ca_fp8_paged_attention (the same kernels),
 * with the decode's partials held in a scratch array of the library
 * (CA_NOALLOC_SCRATCH_BYTES per device, kept from the library's load until
 * the process ends). No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Sizes whose partials exceed the
 * scratch return CA_INVALID_ARGUMENT. The partials are those of the launch's
 * plan: for fp16/bf16 queries, when the longest context spans more than 128
 * blocks, num_seqs <= 1024 and the balanced walk's partials fit the
 * workspace ca_decode_workspace_bytes names, 2 * (4 * compute units) *
 * min(16, num_q_heads / num_kv_heads) * (head_dim + 1) * 4 + 4 * num_seqs
 * bytes (4.2 MB at head dim 128 and 4 query heads per kv head on a
 * 256-CU device, whatever the context lengths); otherwise num_seqs *
 * num_q_heads * splits * (head_dim + 1) * 4 bytes with splits =
 * ceil(max_blocks_per_seq / 128) for fp16/bf16 queries and
 * ceil(max_blocks_per_seq / 64) for float32 (none when that is 1). Every
 * call on a device shares that device's scratch,
 * so the calls are serialised on the device: a call on another stream than
 * the previous call's waits (on the GPU, through an event) for that call's
 * kernels, and concurrent host threads take turns. Under stream capture that
 * wait is left out and the order of the graph launches is the caller's. */
#define CA_NOALLOC_SCRATCH_BYTES (16u << 20)
ca_status ca_fp8_paged_attention_noalloc(ca_dtype dtype, const void* query,
                                         const uint8_t* key_cache, const uint8_t* value_cache,
                                         const float* k_scale, const float* v_scale,
                                         int per_block_scales, const int32_t* block_tables,
                                         const int32_t* context_lens, void* out, int num_seqs,
                                         int num_q_heads, int num_kv_heads, int head_dim,
                                         int max_blocks_per_seq, int page_size, int num_blocks,
                                         float softmax_scale, void* stream);

/* Scale formats of the MXFP8 entry point: e8m0 bytes (the MX storage
 * format, value 2^(byte - 127), 0xFF = NaN) or float32 powers of two (the
 * reference's `const float*` form, kernels_api.h:103-108). */
typedef enum CA_ENUM_INT { CA_SCALE_E8M0 = 0, CA_SCALE_F32 = 1 } ca_scale_kind;

/* MXFP8 attention: q, k, v are OCP e4m3 codes [batch, num_heads, seq_len,
 * head_dim] with one scale per 32 elements along head_dim ([batch, num_heads,
 * seq_len, head_dim / 32], in scale_kind's format); value = code * scale.
 * Output [batch, num_heads, seq_len, head_dim] in out_dtype (CA_BF16 or
 * CA_F16). head_dim must be 128. q_scale and k_scale must be 4-byte aligned
 * (with CA_SCALE_F32 so must v_scale). Limits: a finite softmax_scale, seq_len
 * below 2^22 and batch * num_heads * seq_len below 2^30 (else
 * CA_INVALID_ARGUMENT, before anything is launched). Replaces
 * dispatch_fused_microscaled_attention<T_OUT> (kernels_api.h:103-108).
 * workspace: ca_mx_workspace_bytes(...) (v dequantised to bf16; with float
 * scales also q's and k's converted scale bytes). Asynchronous in both scale
 * forms, like the other entry points: with CA_SCALE_F32 a scale that is not a
 * power of two in [2^-127, 2^127] is taken as the e8m0 NaN, so the outputs it
 * reaches are not meaningful (NaN, or 0 for a row whose logits are all NaN);
 * ca_check_mx_scales reports such scales. */
ca_status ca_fused_microscaled_attention(ca_dtype out_dtype, const uint8_t* q, const void* q_scale,
                                         const uint8_t* k, const void* k_scale, const uint8_t* v,
                                         const void* v_scale, ca_scale_kind scale_kind, void* out,
                                         int batch, int num_heads, int seq_len, int head_dim,
                                         float softmax_scale, int is_causal, void* workspace,
                                         size_t workspace_bytes, void* stream);

/* Bytes of the ca_fused_microscaled_attention workspace (0 for an invalid
 * shape or scale kind). */
size_t ca_mx_workspace_bytes(ca_scale_kind scale_kind, int batch, int num_heads, int seq_len,
                             int head_dim);

/* Debug check of float MX scales (no counterpart in the reference, whose
 * kernels_api.h:103-108 takes the scales unchecked): returns
 * CA_INVALID_ARGUMENT if any entry of q_scale, k_scale or v_scale ([batch,
 * num_heads, seq_len, head_dim / 32] float32 each) is not a power of two in
 * [2^-127, 2^127], which ca_fused_microscaled_attention would take as NaN.
 * Synchronous: it waits for `stream`; it allocates a 4-byte flag. */
ca_status ca_check_mx_scales(const float* q_scale, const float* k_scale, const float* v_scale,
                             int batch, int num_heads, int seq_len, int head_dim, void* stream);

/* Debug check of a paged-cache block table (no counterpart in the reference,
 * which reads through the table unchecked, paged_attention_kernel.cuh:69):
 * returns CA_INVALID_ARGUMENT, naming the first offender, if an entry that a
 * sequence uses (index < ceil(context_lens[n] / page_size), within the
 * table's width) lies outside [0, num_blocks). The paged decode entry points
 * clamp such ids instead, so a corrupt table gives plausible but wrong
 * output; callers that want the error run this first. Synchronous: it waits
 * for `stream` and copies the table and lengths to the host. */
ca_status ca_check_block_tables(const int32_t* block_tables, const int32_t* context_lens,
                                int num_seqs, int max_blocks_per_seq, int num_blocks,
                                int page_size, void* stream);

/* Bytes of workspace the decode entry points need (0 if none). max_tokens is
 * kv_len for ca_flash_decode and max_blocks_per_seq * page_size for the paged
 * entry points. No counterpart in the reference (its decode is not split). */
size_t ca_decode_workspace_bytes(int num_seqs, int num_q_heads, int head_dim, int max_tokens);

/* Thread-local description of the last non-OK status of this thread. */
const char* ca_last_error(void);

/* Library version string. */
const char* ca_version(void);

#ifdef __cplusplus
}
#endif

#endif /* CUDA_LLM_ABI_H */
