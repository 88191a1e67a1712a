"""The reference's attention-forward Python API, on the gfx950 C ABI.

Mirrors the pybind11 module of the reference (fused_softmax_binding.cpp:721-809)
and the ``cuda_llm`` names of its README (README.md:64-81): same function
names, argument names, defaults and error type (``RuntimeError``, which is
what a failed ``TORCH_CHECK`` raises). Outputs are allocated with the torch
caching allocator and every kernel runs on the current HIP stream.

Differences from the reference, all widening what is accepted:
  * GQA: k/v (or the caches) may have fewer heads than q when they divide it
    (kv head = q head // (Hq / Hkv), tests/_utils.py:67-72);
  * FP8 caches decode OCP e4m3, the reference test's intended semantics
    (tests/test_kernels_misc.py:42-64), and also accept float8_e4m3fn tensors;
  * a sequence with context length 0 yields zeros instead of an unwritten row.
float32 q/k/v are accepted where the reference instantiates float (prefill,
flash_decode, paged decode). ``flash_attention`` is differentiable (README.md:
66-71) through ``flash_attention_backward`` (fp16 / bf16 / float32, as the
reference instantiates it).
"""
import ctypes
import math
import os

import torch

from . import _lib

__all__ = [
    "flash_attention", "flash_attention_forward", "flash_attention_v3_hopper",
    "flash_attention_forward_lse", "flash_attention_backward",
    "fused_gqa_forward", "fused_rope_flash_attention", "flash_decode", "async_flash_decode", "paged_attention",
    "paged_attention_forward", "fp8_paged_attention", "fp8_paged_attention_forward",
    "fused_microscaled_attention", "mx_scales_to_e8m0", "paged_kv_append",
]

_DT = {torch.bfloat16: _lib.CA_BF16, torch.float16: _lib.CA_F16, torch.float32: _lib.CA_F32}
_FP8_CACHE_DTYPES = (torch.uint8, torch.int8, torch.float8_e4m3fn)


def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


if hasattr(torch._C, "_cuda_getCurrentRawStream") and hasattr(torch._C, "_cuda_getDevice"):
    def _stream():
        # The current device's current stream, as torch.cuda.current_stream()
        # gives it, without building a Stream object (0.3 us instead of 3 us
        # per call on the host).
        return ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(torch._C._cuda_getDevice()))
else:
    def _stream():
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _aligned(t):
    """Contiguous tensor whose storage pointer is 16-byte aligned."""
    if t.data_ptr() % 16 == 0:
        return t
    return t.clone()


def _scale(softmax_scale, head_dim):
    # fused_softmax_binding.cpp:69-72
    return float(softmax_scale) if softmax_scale is not None else 1.0 / math.sqrt(head_dim)


def _dtype_code(t, what):
    _check(t.dtype in _DT, f"Unsupported scalar type for {what}. Supported: Float, Float16, BFloat16.")
    return _DT[t.dtype]


def _workspace(nbytes, device):
    if nbytes == 0:
        return None, 0
    return torch.empty(nbytes, dtype=torch.uint8, device=device), nbytes


# ---------------------------------------------------------------------------
# Prefill
# ---------------------------------------------------------------------------
def _prefill_checks(q, k, v):
    _check(q.is_cuda and k.is_cuda and v.is_cuda, "Inputs must be on CUDA")
    _check(q.is_contiguous() and k.is_contiguous() and v.is_contiguous(),
           "Inputs must be contiguous")
    _check(q.dim() == 4, "Expected 4D tensor: [batch, num_heads, seq_len, head_dim]")
    _check(k.dim() == 4 and v.dim() == 4 and k.shape == v.shape,
           "Q, K, V must have identical shapes")
    b, hq, s, d = q.shape
    _check(k.shape[0] == b and k.shape[2] == s and k.shape[3] == d and k.shape[1] >= 1
           and hq % k.shape[1] == 0, "Q, K, V must have identical shapes "
           "(or K/V with a number of heads dividing Q's)")
    _check(q.dtype == k.dtype == v.dtype, "Q, K, V must have the same dtype")
    _check(d in (64, 128), "Only head_dim 64 and 128 are currently supported")


def flash_attention_forward(q, k, v, is_causal=False, softmax_scale=None):
    """O = softmax(Q K^T * scale [+ causal]) V.

    q: [B, Hq, S, D]; k, v: [B, Hkv, S, D] (Hkv == Hq in the reference; any
    divisor of Hq here). Reference: fused_softmax_binding.cpp:49-103.
    """
    _prefill_checks(q, k, v)
    b, hq, s, d = q.shape
    dt = _dtype_code(q, "FlashAttention")
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    out = torch.empty_like(q)
    _lib.call("ca_flash_attention_fwd", dt, _ptr(q), _ptr(k), _ptr(v), _ptr(out), b, hq,
              k.shape[1], s, d, _scale(softmax_scale, d), int(bool(is_causal)), _stream())
    return out


def flash_attention_forward_lse(q, k, v, is_causal=False, softmax_scale=None):
    """(O, LSE): the prefill forward plus the natural-log logsumexp of every
    row of scaled, masked scores, LSE [B, Hq, S] float32 (-inf for a row with
    no visible key). No reference counterpart: the reference's forward returns
    O only; its backward takes this LSE (fused_softmax_binding.cpp:367-376),
    which its tests build with ref_lse (tests/_utils.py:56-64)."""
    _prefill_checks(q, k, v)
    b, hq, s, d = q.shape
    dt = _dtype_code(q, "FlashAttention")
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    out = torch.empty_like(q)
    lse = torch.empty(b, hq, s, dtype=torch.float32, device=q.device)
    _lib.call("ca_flash_attention_fwd_lse", dt, _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(lse),
              b, hq, k.shape[1], s, d, _scale(softmax_scale, d), int(bool(is_causal)), _stream())
    return out, lse


def flash_attention_backward(dout, q, k, v, out, lse, is_causal=False, softmax_scale=None):
    """[dq, dk, dv] of O = softmax(Q K^T * scale [+ causal]) V, given the
    forward output ``out``, its gradient ``dout`` and the forward's
    natural-log row logsumexp ``lse`` [B, Hq, S] (fused_softmax_binding.cpp:
    367-433; math flash_attention_bwd_kernel.cuh:9-19). q, out, dout: [B, Hq,
    S, D]; k, v: [B, Hkv, S, D] (GQA: dk, dv sum over the q heads of a kv
    head). fp16 / bf16 / float32; lse is converted to contiguous float32 as
    the reference does."""
    _check(dout.is_cuda and q.is_cuda and k.is_cuda and v.is_cuda and out.is_cuda,
           "Inputs must be on CUDA")
    _check(lse.is_cuda, "LSE tensor must be on CUDA")
    _check(q.dim() == 4, "Expected 4D tensor: [batch, num_heads, seq_len, head_dim]")
    b, hq, s, d = q.shape
    _check(k.dim() == 4 and v.dim() == 4 and k.shape == v.shape and k.shape[0] == b
           and k.shape[2] == s and k.shape[3] == d and hq % k.shape[1] == 0,
           "K, V must be [batch, num_kv_heads, seq_len, head_dim] with num_kv_heads dividing "
           "Q's heads")
    _check(dout.shape == q.shape and out.shape == q.shape, "dout and out must have Q's shape")
    _check(lse.shape == (b, hq, s), "lse must be [batch, num_heads, seq_len]")
    _check(q.dtype == k.dtype == v.dtype == out.dtype == dout.dtype,
           "q, k, v, out and dout must have the same dtype")
    _check(d in (64, 128), "Only head_dim 64 and 128 are currently supported")
    _check(q.dtype in _DT,
           "Unsupported scalar type for FlashAttention Backward. Supported: Float, Float16, "
           "BFloat16.")
    dt = _DT[q.dtype]
    q, k, v, out, dout = (_aligned(t.contiguous()) for t in (q, k, v, out, dout))
    lse = lse.to(torch.float32).contiguous()
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws, nbytes = _workspace(int(_lib.load().ca_flash_attention_bwd_workspace_bytes(b, hq, s)),
                            q.device)
    _lib.call("ca_flash_attention_bwd", dt, _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(dout),
              _ptr(lse), _ptr(dq), _ptr(dk), _ptr(dv), b, hq, k.shape[1], s, d,
              _scale(softmax_scale, d), int(bool(is_causal)), _ptr(ws), nbytes, _stream())
    return [dq, dk, dv]


class _FlashAttention(torch.autograd.Function):
    """Autograd node: forward with LSE, backward through flash_attention_backward."""

    @staticmethod
    def forward(ctx, q, k, v, is_causal, softmax_scale):
        out, lse = flash_attention_forward_lse(q, k, v, is_causal, softmax_scale)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.is_causal, ctx.softmax_scale = is_causal, softmax_scale
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        dq, dk, dv = flash_attention_backward(dout.contiguous(), q, k, v, out, lse,
                                              ctx.is_causal, ctx.softmax_scale)
        return dq, dk, dv, None, None


def flash_attention(q, k, v, is_causal=False, softmax_scale=None):
    """README's ``cllm.flash_attention`` (README.md:66-71): the prefill forward,
    differentiable with respect to q, k and v when any of them requires grad
    (then the forward also keeps its LSE for the backward kernels)."""
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        return _FlashAttention.apply(q, k, v, is_causal, softmax_scale)
    return flash_attention_forward(q, k, v, is_causal=is_causal, softmax_scale=softmax_scale)


flash_attention_v3_hopper = flash_attention_forward


def fused_gqa_forward(q, k, v, is_causal=True, softmax_scale=None):
    """GQA prefill (fused_softmax_binding.cpp:246-302; default causal)."""
    return flash_attention_forward(q, k, v, is_causal=is_causal, softmax_scale=softmax_scale)


def fused_rope_flash_attention(q, k, v, cos_tab, sin_tab, is_causal=True, softmax_scale=None):
    """Prefill on RoPE-rotated q and k (fused_softmax_binding.cpp:179-241):
    rotate-half convention, cos_tab / sin_tab [seq_len, head_dim] (converted
    to contiguous float32 as the reference does); q, k, v as
    flash_attention_forward (GQA allowed)."""
    _check(cos_tab.is_cuda and sin_tab.is_cuda, "RoPE tables must be on CUDA")
    _prefill_checks(q, k, v)
    b, hq, s, d = q.shape
    _check(tuple(cos_tab.shape) == (s, d) and tuple(sin_tab.shape) == (s, d),
           "RoPE tables must be [seq_len, head_dim]")
    dt = _dtype_code(q, "Fused RoPE Attention")
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    cos_f, sin_f = (_aligned(t.to(torch.float32).contiguous()) for t in (cos_tab, sin_tab))
    out = torch.empty_like(q)
    hkv = k.shape[1]
    ws, nbytes = _workspace(int(_lib.load().ca_rope_workspace_bytes(dt, b, hq, hkv, s, d)), q.device)
    _lib.call("ca_fused_rope_flash_attention", dt, _ptr(q), _ptr(k), _ptr(v), _ptr(cos_f),
              _ptr(sin_f), _ptr(out), b, hq, hkv, s, d, _scale(softmax_scale, d),
              int(bool(is_causal)), _ptr(ws), nbytes, _stream())
    return out


# ---------------------------------------------------------------------------
# Decode over a contiguous cache
# ---------------------------------------------------------------------------
def async_flash_decode(q, k, v, softmax_scale=None):
    """q: [B, Hq, 1, D]; k, v: [B, Hkv, S_kv, D] -> [B, Hq, 1, D].
    Reference: fused_softmax_binding.cpp:308-360."""
    _check(q.is_cuda and k.is_cuda and v.is_cuda, "Inputs must be on CUDA")
    _check(q.dim() == 4 and k.dim() == 4 and v.dim() == 4,
           "Inputs must be 4D [batch, heads, seq, dim]")
    _check(q.size(2) == 1, "Query sequence length must be 1 for Flash-Decoding")
    _check(k.shape == v.shape, "K and V must have identical shapes")
    b, hq, _, d = q.shape
    _check(k.size(0) == b and k.size(3) == d and hq % k.size(1) == 0,
           "K/V batch and head_dim must match Q; Q heads must be a multiple of K/V heads")
    _check(d in (64, 128), "Only head_dim 64 and 128 supported")
    _check(q.dtype == k.dtype == v.dtype, "Q, K, V must have the same dtype")
    dt = _dtype_code(q, "Async Flash-Decode")
    q, k, v = (_aligned(t.contiguous()) for t in (q, k, v))
    hkv, s_kv = k.size(1), k.size(2)
    out = torch.empty_like(q)
    ws, nbytes = _workspace(_lib.load().ca_decode_workspace_bytes(b, hq, d, s_kv), q.device)
    _lib.call("ca_flash_decode", dt, _ptr(q), _ptr(k), _ptr(v), _ptr(out), b, hq, hkv, s_kv, d,
              _scale(softmax_scale, d), _ptr(ws), nbytes, _stream())
    return out


flash_decode = async_flash_decode


# ---------------------------------------------------------------------------
# Paged decode
# ---------------------------------------------------------------------------
def _paged_checks(query, key_cache, value_cache, block_tables, context_lens):
    _check(query.is_cuda and key_cache.is_cuda and value_cache.is_cuda, "Inputs must be on CUDA")
    _check(block_tables.is_cuda and context_lens.is_cuda, "Metadata tensors must be on CUDA")
    _check(query.dim() == 3, "Query must be 3D [num_seqs, num_heads, head_dim]")
    _check(key_cache.dim() == 4 and value_cache.dim() == 4,
           "KV caches must be 4D [num_blocks, num_heads, head_dim, page_size]")
    _check(key_cache.shape == value_cache.shape, "K and V caches must have identical shapes")
    n, hq, d = query.shape
    _check(d in (64, 128), "Only head_dim 64 and 128 supported")
    _check(key_cache.size(2) == d, "Cache head_dim must match the query's")
    _check(key_cache.size(3) == 16, "Only page_size 16 is currently supported")
    hkv = key_cache.size(1)
    _check(hkv >= 1 and hq % hkv == 0, "Query heads must be a multiple of cache heads")
    _check(block_tables.dim() == 2 and block_tables.size(0) == n,
           "block_tables must be [num_seqs, max_blocks_per_seq]")
    _check(context_lens.dim() == 1 and context_lens.size(0) == n, "context_lens must be [num_seqs]")
    _check(block_tables.dtype == torch.int32 and context_lens.dtype == torch.int32,
           "block_tables and context_lens must be int32")
    return n, hq, hkv, d


def _debug_check_tables(block_tables, context_lens, num_blocks):
    """With CUDA_LLM_CHECK_BLOCK_TABLES=1 in the environment, every paged call
    first checks that the table entries its sequences use lie in the pool
    (ca_check_block_tables, synchronous) and raises RuntimeError otherwise;
    by default ids outside the pool are clamped by the kernels."""
    if os.environ.get("CUDA_LLM_CHECK_BLOCK_TABLES", "0") not in ("", "0"):
        _lib.call("ca_check_block_tables", _ptr(block_tables), _ptr(context_lens),
                  block_tables.size(0), block_tables.size(1), num_blocks, 16, _stream())


def paged_attention_forward(query, key_cache, value_cache, block_tables, context_lens,
                            softmax_scale=None):
    """vLLM-style paged decode (fused_softmax_binding.cpp:109-173).

    query [N, Hq, D]; caches [num_blocks, Hkv, D, 16] of the query dtype;
    block_tables int32 [N, max_blocks]; context_lens int32 [N] -> [N, Hq, D].
    """
    n, hq, hkv, d = _paged_checks(query, key_cache, value_cache, block_tables, context_lens)
    _check(key_cache.dtype == query.dtype and value_cache.dtype == query.dtype,
           "Caches must have the query dtype")
    dt = _dtype_code(query, "PagedAttention")
    query, key_cache, value_cache = (_aligned(t.contiguous()) for t in (query, key_cache, value_cache))
    block_tables, context_lens = block_tables.contiguous(), context_lens.contiguous()
    _debug_check_tables(block_tables, context_lens, key_cache.size(0))
    out = torch.empty_like(query)
    max_blocks = block_tables.size(1)
    ws, nbytes = _workspace(_lib.load().ca_decode_workspace_bytes(n, hq, d, max_blocks * 16),
                            query.device)
    _lib.call("ca_paged_attention", dt, _ptr(query), _ptr(key_cache), _ptr(value_cache),
              _ptr(block_tables), _ptr(context_lens), _ptr(out), n, hq, hkv, d, max_blocks, 16,
              key_cache.size(0), _scale(softmax_scale, d), _ptr(ws), nbytes, _stream())
    return out


paged_attention = paged_attention_forward


def fp8_paged_attention_forward(query, key_cache_fp8, value_cache_fp8, k_scale, v_scale,
                                block_tables, context_lens, softmax_scale=None):
    """FP8 (e4m3) paged decode (fused_softmax_binding.cpp:634-718).

    Caches: e4m3 codes as uint8 / int8 / float8_e4m3fn [num_blocks, Hkv, D, 16].
    Scales: fp32-convertible, [Hkv] per head or [num_blocks, Hkv] per block
    (``k_scale.dim() == 2`` selects per-block, :671). Output in query dtype.
    """
    _check(k_scale.is_cuda and v_scale.is_cuda, "Scale tensors must be on CUDA")
    n, hq, hkv, d = _paged_checks(query, key_cache_fp8, value_cache_fp8, block_tables, context_lens)
    _check(key_cache_fp8.dtype in _FP8_CACHE_DTYPES and value_cache_fp8.dtype in _FP8_CACHE_DTYPES,
           "KV caches must be 8-bit quantized (int8 or uint8)")
    dt = _dtype_code(query, "FP8 PagedAttention")
    per_block = k_scale.dim() == 2
    num_blocks = key_cache_fp8.size(0)
    if per_block:
        _check(tuple(k_scale.shape) == (num_blocks, hkv) and tuple(v_scale.shape) == (num_blocks, hkv),
               "per-block scales must be [num_blocks, num_kv_heads]")
    else:
        _check(k_scale.numel() == hkv and v_scale.numel() == hkv,
               "per-head scales must be [num_kv_heads]")
    k_scale = k_scale.to(torch.float32).contiguous()
    v_scale = v_scale.to(torch.float32).contiguous()
    query = _aligned(query.contiguous())
    kc = _aligned(key_cache_fp8.contiguous())
    vc = _aligned(value_cache_fp8.contiguous())
    block_tables, context_lens = block_tables.contiguous(), context_lens.contiguous()
    _debug_check_tables(block_tables, context_lens, num_blocks)
    out = torch.empty_like(query)
    max_blocks = block_tables.size(1)
    ws, nbytes = _workspace(_lib.load().ca_decode_workspace_bytes(n, hq, d, max_blocks * 16),
                            query.device)
    _lib.call("ca_fp8_paged_attention", dt, _ptr(query), _ptr(kc), _ptr(vc), _ptr(k_scale),
              _ptr(v_scale), int(per_block), _ptr(block_tables), _ptr(context_lens), _ptr(out),
              n, hq, hkv, d, max_blocks, 16, num_blocks, _scale(softmax_scale, d), _ptr(ws),
              nbytes, _stream())
    return out


fp8_paged_attention = fp8_paged_attention_forward


def paged_kv_append(key, value, key_cache, value_cache, block_tables, context_lens,
                    new_lens=None, k_scale=None, v_scale=None):
    """Append new tokens to a paged KV cache in place (the step before paged
    decode; no reference kernel: its tests build caches in torch, tests/
    _utils.py:105-133, in the layout the paged decode entry points read).

    key, value: [N, Hkv, T, D] fp16/bf16. Sequence n appends its first
    ``new_lens[n]`` tokens (default T) at positions ``context_lens[n]`` ..
    through ``block_tables`` [N, max_blocks]; ``context_lens`` is not updated.
    Caches [num_blocks, Hkv, D, 16]: of key's dtype, or e4m3 codes (uint8 /
    int8 / float8_e4m3fn) with float32 ``k_scale``/``v_scale``: per head [Hkv]
    (new slots quantised with the given scale, saturated to +-448) or per
    (page, head) [num_blocks, Hkv] (every touched page quantised again with
    scale = max(amax / 448, 1e-8), written in place; tests/test_kernels_misc.
    py:52-55 per page). Positions past the table and block ids outside the
    pool are skipped.
    """
    _check(key.is_cuda and value.is_cuda and key_cache.is_cuda and value_cache.is_cuda,
           "Inputs must be on CUDA")
    _check(block_tables.is_cuda and context_lens.is_cuda, "Metadata tensors must be on CUDA")
    _check(key.dim() == 4 and key.shape == value.shape,
           "key and value must be [num_seqs, num_kv_heads, new_tokens, head_dim]")
    n, hkv, t, d = key.shape
    _check(key_cache.dim() == 4 and key_cache.shape == value_cache.shape
           and key_cache.size(1) == hkv and key_cache.size(2) == d and key_cache.size(3) == 16,
           "caches must be [num_blocks, num_kv_heads, head_dim, 16]")
    _check(key_cache.is_contiguous() and value_cache.is_contiguous(),
           "caches must be contiguous (they are written in place)")
    _check(block_tables.dim() == 2 and block_tables.size(0) == n, "block_tables must be [num_seqs, max_blocks]")
    _check(context_lens.numel() == n, "context_lens must have num_seqs entries")
    _check(key.dtype == value.dtype, "key and value must have the same dtype")
    dt = _dtype_code(key, "paged_kv_append")
    _check(dt != _lib.CA_F32, "paged_kv_append: key/value must be fp16 or bf16")
    fp8 = key_cache.dtype in _FP8_CACHE_DTYPES
    num_blocks = key_cache.size(0)
    per_block = False
    if fp8:
        _check(value_cache.dtype in _FP8_CACHE_DTYPES, "both caches must be FP8")
        _check(k_scale is not None and v_scale is not None, "FP8 caches need k_scale and v_scale")
        _check(k_scale.is_cuda and v_scale.is_cuda, "Scale tensors must be on CUDA")
        _check(k_scale.dtype == torch.float32 and v_scale.dtype == torch.float32
               and k_scale.is_contiguous() and v_scale.is_contiguous(),
               "scales must be contiguous float32 (per-page scales are written in place)")
        per_block = k_scale.dim() == 2
        if per_block:
            _check(tuple(k_scale.shape) == (num_blocks, hkv) and tuple(v_scale.shape) == (num_blocks, hkv),
                   "per-block scales must be [num_blocks, num_kv_heads]")
        else:
            _check(k_scale.numel() == hkv and v_scale.numel() == hkv,
                   "per-head scales must be [num_kv_heads]")
    else:
        _check(key_cache.dtype == key.dtype and value_cache.dtype == key.dtype,
               "16-bit caches must have key's dtype")
    key, value = (_aligned(x.contiguous()) for x in (key, value))
    tables = block_tables.to(torch.int32).contiguous()
    lens = context_lens.to(torch.int32).contiguous()
    nl = None
    if new_lens is not None:
        _check(new_lens.is_cuda and new_lens.numel() == n, "new_lens must be [num_seqs] on CUDA")
        nl = new_lens.to(torch.int32).contiguous()
    _lib.call("ca_paged_kv_append", dt, int(fp8), _ptr(key), _ptr(value), _ptr(key_cache),
              _ptr(value_cache), _ptr(k_scale if fp8 else None), _ptr(v_scale if fp8 else None),
              int(per_block), _ptr(tables), _ptr(lens), _ptr(nl), n, hkv, d, t,
              tables.size(1), num_blocks, _stream())


# ---------------------------------------------------------------------------
# MXFP8
# ---------------------------------------------------------------------------
def mx_scales_to_e8m0(scale):
    """MX block scales -> uint8 e8m0 bytes on the same device.

    Accepts uint8 / float8_e8m0fnu (returned as uint8 views) or floating
    tensors holding exact powers of two (converted; anything else raises,
    because an MX scale is a pure power of two).
    """
    if scale.dtype == torch.uint8:
        return scale
    if scale.dtype == torch.float8_e8m0fnu:
        return scale.view(torch.uint8)
    _check(scale.is_floating_point(), "MX scales must be e8m0 bytes or float powers of two")
    s = scale.to(torch.float32)
    mant, exp = torch.frexp(s)
    _check(bool(((mant == 0.5) & (exp - 1 >= -127) & (exp - 1 <= 127)).all()),
           "float MX scales must be powers of two in [2^-127, 2^127]")
    return (exp - 1 + 127).to(torch.uint8)


def fused_microscaled_attention(q_fp8, q_scale, k_fp8, k_scale, v_fp8, v_scale,
                                is_causal=False, softmax_scale=None, out_dtype=torch.bfloat16):
    """Attention over MXFP8 q/k/v (README.md:29-31,80-81; kernels_api.h:103-108).

    q/k/v: e4m3 codes (uint8 / int8 / float8_e4m3fn) [B, H, S, 128];
    scales: one per 32 elements along D, [B, H, S, 4]: e8m0 bytes (uint8 /
    float8_e8m0fnu) or floating tensors holding powers of two (the
    reference's float form; passed to the C ABI as float32, which takes
    anything else as NaN; with CUDA_LLM_CHECK_MX_SCALES=1 in the environment
    they are checked first, synchronously, and RuntimeError is raised).
    Mixed forms are brought to e8m0 bytes here, which checks them. Output
    [B, H, S, 128] bf16/fp16.
    """
    for t in (q_fp8, k_fp8, v_fp8, q_scale, k_scale, v_scale):
        _check(t.is_cuda, "Inputs must be on CUDA")
    _check(q_fp8.dim() == 4, "Expected 4D tensor: [batch, num_heads, seq_len, head_dim]")
    _check(q_fp8.shape == k_fp8.shape == v_fp8.shape, "Q, K, V must have identical shapes")
    for t in (q_fp8, k_fp8, v_fp8):
        _check(t.dtype in _FP8_CACHE_DTYPES, "MXFP8 codes must be uint8, int8 or float8_e4m3fn")
    b, h, s, d = q_fp8.shape
    _check(d == 128, "MXFP8 attention supports head_dim 128")
    for sc in (q_scale, k_scale, v_scale):
        _check(tuple(sc.shape) == (b, h, s, d // 32), "MX scales must be [B, H, S, head_dim/32]")
    _check(out_dtype in (torch.bfloat16, torch.float16), "out_dtype must be bfloat16 or float16")
    scales = (q_scale, k_scale, v_scale)
    if all(t.is_floating_point() and t.dtype != torch.float8_e8m0fnu for t in scales):
        kind = _lib.CA_SCALE_F32
        qs, ks, vs = (_aligned(t.to(torch.float32).contiguous()) for t in scales)
        if os.environ.get("CUDA_LLM_CHECK_MX_SCALES", "0") not in ("", "0"):
            # ca_check_mx_scales (synchronous): by default a scale that is not
            # a power of two is taken as NaN and the call stays asynchronous
            _lib.call("ca_check_mx_scales", _ptr(qs), _ptr(ks), _ptr(vs), b, h, s, d, _stream())
    else:
        kind = _lib.CA_SCALE_E8M0
        qs, ks, vs = (mx_scales_to_e8m0(t).contiguous() for t in scales)
        ks = _aligned(ks)
    q8, k8, v8 = (_aligned(t.contiguous()) for t in (q_fp8, k_fp8, v_fp8))
    out = torch.empty((b, h, s, d), dtype=out_dtype, device=q_fp8.device)
    ws, nbytes = _workspace(int(_lib.load().ca_mx_workspace_bytes(kind, b, h, s, d)), q_fp8.device)
    _lib.call("ca_fused_microscaled_attention", _DT[out_dtype], _ptr(q8), _ptr(qs), _ptr(k8),
              _ptr(ks), _ptr(v8), _ptr(vs), kind, _ptr(out), b, h, s, d, _scale(softmax_scale, d),
              int(bool(is_causal)), _ptr(ws), nbytes, _stream())
    return out
