"""GPU tier: float32 inputs (prefill, flash_decode, paged and FP8 paged
decode) vs the oracle.

The reference binding dispatches float32 for flash_attention / _v3_hopper /
fused_gqa (fused_softmax_binding.cpp:77-81, 275-277), async_flash_decode,
paged_attention (:142-146) and fp8_paged_attention with float queries
(:683-691, instantiated at fp8_paged_attention_instantiations.cu:4); its tests
use fp16/bf16 only (tests/test_attention.py:13 there), so the grids below are
its fp16/bf16 grids run in float32, plus split-K lengths, ragged S, the golden
vectors, NaN bytes past a paged context's end and BASELINE config C1 (fp32
causal B=2 H=8 S=1024 D=64, the workload of tests/_utils.py:48-53 there).
Tolerance: the reference's float32 tolerance (tests/_utils.py:23-27 there,
1e-4), here as max-abs 1e-4 and mean-abs 1e-5 against the float64 oracle (for
FP8 caches: on the dequantised codes, so only fp32 arithmetic separates the
two).
"""
import os

import numpy as np
import pytest
import torch

import cuda_llm
import oracle
from _util import assert_close, build_paged, paged_oracle, qkv, to_np

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
TOL_F32 = dict(max_abs=1e-4, mean_abs=1e-5)
F32 = torch.float32


@pytest.mark.parametrize("fn_name", ["flash_attention_forward", "flash_attention_v3_hopper"])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("seq_len", [1, 64, 100, 256, 300])
@pytest.mark.parametrize("is_causal", [False, True])
def test_flash_forward_f32(dev, fn_name, head_dim, seq_len, is_causal):
    q, k, v = qkv(2, 4, seq_len, head_dim, F32, dev)
    out = getattr(cuda_llm, fn_name)(q, k, v, is_causal=is_causal)
    torch.cuda.synchronize()
    assert out.dtype == F32
    ref = oracle.attention(to_np(q), to_np(k), to_np(v), is_causal=is_causal, dtype=np.float64)
    assert_close(to_np(out), ref, **TOL_F32, name=fn_name)


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("hq,hkv", [(8, 2), (8, 8), (4, 1)])
@pytest.mark.parametrize("is_causal", [False, True])
def test_gqa_f32(dev, head_dim, hq, hkv, is_causal):
    q, k, v = qkv(1, hq, 100, head_dim, F32, dev, hkv=hkv)
    out = cuda_llm.fused_gqa_forward(q, k, v, is_causal=is_causal)
    torch.cuda.synchronize()
    ref = oracle.attention(to_np(q), to_np(k), to_np(v), is_causal=is_causal, dtype=np.float64)
    assert_close(to_np(out), ref, **TOL_F32, name="gqa f32")


@pytest.mark.parametrize("name", ["attn_causal_d64", "attn_full_d64", "attn_gqa_causal_d128"])
def test_golden_vectors_f32(dev, name):
    g = np.load(GOLDEN, allow_pickle=False)
    q, k, v = (torch.from_numpy(g[f"{name}/{x}"]).to(dev).to(F32) for x in "qkv")
    out = cuda_llm.flash_attention(q, k, v, is_causal=bool(g[f"{name}/causal"]))
    torch.cuda.synchronize()
    assert_close(to_np(out), g[f"{name}/out"], **TOL_F32, name=name)


def test_large_logits_and_negative_scale_f32(dev):
    q, k, v = qkv(1, 2, 200, 128, F32, dev)
    q = q * 8.0
    for scale in (0.5, -0.2):
        out = cuda_llm.flash_attention(q, k, v, is_causal=True, softmax_scale=scale)
        torch.cuda.synchronize()
        ref = oracle.attention(to_np(q), to_np(k), to_np(v), is_causal=True, scale=scale,
                               dtype=np.float64)
        assert_close(to_np(out), ref, **TOL_F32, name=f"scale {scale}")


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("kv_len", [1, 63, 64, 1000, 2500])
def test_flash_decode_f32(dev, head_dim, kv_len):
    q = torch.randn(2, 4, 1, head_dim, device=dev, dtype=F32)
    k = torch.randn(2, 4, kv_len, head_dim, device=dev, dtype=F32)
    v = torch.randn(2, 4, kv_len, head_dim, device=dev, dtype=F32)
    out = cuda_llm.async_flash_decode(q, k, v)
    torch.cuda.synchronize()
    ref = oracle.attention(to_np(q), to_np(k), to_np(v), dtype=np.float64)
    assert_close(to_np(out), ref, **TOL_F32, name="decode f32")


@pytest.mark.parametrize("hq,hkv,kv_len", [(32, 8, 5000), (8, 1, 1025), (40, 2, 700)])
def test_flash_decode_gqa_split_f32(dev, hq, hkv, kv_len):
    q = torch.randn(2, hq, 1, 128, device=dev, dtype=F32)
    k = torch.randn(2, hkv, kv_len, 128, device=dev, dtype=F32)
    v = torch.randn(2, hkv, kv_len, 128, device=dev, dtype=F32)
    out = cuda_llm.flash_decode(q, k, v)
    torch.cuda.synchronize()
    ref = oracle.attention(to_np(q), to_np(k), to_np(v), dtype=np.float64)
    assert_close(to_np(out), ref, **TOL_F32, name="flash_decode gqa f32")


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("hq,hkv", [(4, 4), (32, 8), (40, 2)])
def test_paged_f32(dev, head_dim, hq, hkv):
    lens = [0, 1, 15, 16, 17, 300, 1023, 1024, 1025, 3000]
    case = build_paged(lens, hq, hkv, head_dim, F32, dev, pool=800)
    out = cuda_llm.paged_attention_forward(case["query"], case["key_cache"], case["value_cache"],
                                           case["block_tables"], case["context_lens"])
    torch.cuda.synchronize()
    assert out.dtype == F32
    assert_close(to_np(out), paged_oracle(case), **TOL_F32, name=f"paged f32 {hq}/{hkv}")
    assert torch.all(out[0] == 0)


def test_paged_f32_nan_tail_does_not_leak(dev):
    """Bytes past a sequence's length in its last page may be anything."""
    case = build_paged([37, 5, 1030], 8, 2, 128, F32, dev)
    ref = paged_oracle(case)
    for i, L in enumerate([37, 5, 1030]):
        blk = int(case["block_tables"][i, (L - 1) // 16])
        case["key_cache"][blk, :, :, L % 16:] = float("nan")
        case["value_cache"][blk, :, :, L % 16:] = float("nan")
    out = cuda_llm.paged_attention_forward(case["query"], case["key_cache"], case["value_cache"],
                                           case["block_tables"], case["context_lens"])
    torch.cuda.synchronize()
    assert_close(to_np(out), ref, **TOL_F32, name="paged f32 nan tail")


@pytest.mark.parametrize("head_dim", [64, 128])
def test_causal_paired_query_tiles_f32(dev, head_dim):
    """A causal grid big enough that each workgroup takes two query tiles of a
    head (n_qt-1-p and p; the middle tiles of two heads): 15 tiles of 128
    rows, sampled heads."""
    q, k, v = qkv(4, 32, 1900, head_dim, F32, dev, hkv=8)
    out = cuda_llm.flash_attention(q, k, v, is_causal=True)
    torch.cuda.synchronize()
    for (bi, hi) in [(0, 0), (3, 17), (3, 31)]:
        kh = hi // 4
        ref = oracle.attention(to_np(q[bi:bi + 1, hi:hi + 1]), to_np(k[bi:bi + 1, kh:kh + 1]),
                               to_np(v[bi:bi + 1, kh:kh + 1]), is_causal=True, dtype=np.float64)
        assert_close(to_np(out[bi:bi + 1, hi:hi + 1]), ref, **TOL_F32, name=f"head {bi},{hi}")


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("b,hq,hkv,s", [(1, 8, 2, 1000), (1, 2, 1, 2047), (3, 1, 1, 993),
                                        (1, 1, 1, 33), (2, 8, 2, 970)])
def test_split_key_walk_f32(dev, head_dim, is_causal, b, hq, hkv, s):
    """Grids of fewer 128-row tiles than CUs: each 32-row query block's key
    walk is split over the four waves of a workgroup and their softmax states
    merged. Walks of 2 to 64 key tiles (16 per wave), even and odd block
    counts (causal pairs and the lone middle block; 2 x 8 x 970 also pairs
    non-causal blocks, 31 of them per head), ragged S, GQA; O and the LSE
    against the oracle, and O identical with and without the LSE store."""
    q, k, v = qkv(b, hq, s, head_dim, F32, dev, hkv=hkv)
    out, lse = cuda_llm.flash_attention_forward_lse(q, k, v, is_causal=is_causal)
    plain = cuda_llm.flash_attention_forward(q, k, v, is_causal=is_causal)
    torch.cuda.synchronize()
    ref = oracle.attention(to_np(q), to_np(k), to_np(v), is_causal=is_causal, dtype=np.float64)
    assert_close(to_np(out), ref, **TOL_F32, name=f"split {b}x{hq}/{hkv}x{s}")
    ref_lse = oracle.attention_lse(to_np(q), to_np(k), is_causal=is_causal, dtype=np.float64)
    assert np.abs(to_np(lse) - ref_lse).max() <= 1e-4
    assert torch.equal(out, plain)


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("s", [300, 1111])
def test_zero_scale_is_running_mean_f32(dev, head_dim, is_causal, s):
    """softmax_scale = 0 weighs every visible key equally: row i is the mean
    of V over keys 0..i (causal) or over all keys, a closed form that needs
    no oracle; every logit is 0, so the split walk's running max never
    rises after its first tile."""
    q, k, v = qkv(2, 3, s, head_dim, F32, dev)
    out = cuda_llm.flash_attention(q, k, v, is_causal=is_causal, softmax_scale=0.0)
    torch.cuda.synchronize()
    v64 = v.double()
    if is_causal:
        ref = v64.cumsum(2) / torch.arange(1, s + 1, device=dev, dtype=torch.float64)[:, None]
    else:
        ref = v64.mean(2, keepdim=True).expand_as(v64)
    assert_close(to_np(out), to_np(ref), **TOL_F32, name=f"zero scale s={s}")


@pytest.mark.parametrize("head_dim", [64, 128])
def test_full_grid_noncausal_f32(dev, head_dim):
    """A non-causal grid with a 128-row tile for every CU and more (2 x 16
    heads x 9 tiles): the unsplit kernel, sampled heads."""
    q, k, v = qkv(2, 16, 1100, head_dim, F32, dev, hkv=4)
    out = cuda_llm.flash_attention(q, k, v, is_causal=False)
    torch.cuda.synchronize()
    for (bi, hi) in [(0, 0), (1, 9), (1, 15)]:
        kh = hi // 4
        ref = oracle.attention(to_np(q[bi:bi + 1, hi:hi + 1]), to_np(k[bi:bi + 1, kh:kh + 1]),
                               to_np(v[bi:bi + 1, kh:kh + 1]), dtype=np.float64)
        assert_close(to_np(out[bi:bi + 1, hi:hi + 1]), ref, **TOL_F32, name=f"head {bi},{hi}")


def test_baseline_c1(dev):
    """BASELINE configs[0] (C1): fp32 q, k, v ~ N(0,1) [2, 8, 1024, 64], causal,
    scale 1/8, seeded, through cuda_llm.flash_attention."""
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    q, k, v = (torch.randn(2, 8, 1024, 64, device=dev, generator=g) for _ in range(3))
    out = cuda_llm.flash_attention(q, k, v, is_causal=True)
    torch.cuda.synchronize()
    assert out.dtype == F32 and out.shape == q.shape
    ref = oracle.attention(to_np(q), to_np(k), to_np(v), is_causal=True, dtype=np.float64)
    assert_close(to_np(out), ref, **TOL_F32, name="C1")
    # causal row 0 attends to key 0 only: out = v[..., 0, :]
    assert torch.allclose(out[:, :, 0], v[:, :, 0], atol=1e-6, rtol=0)


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("per_block", [False, True])
@pytest.mark.parametrize("hq,hkv", [(4, 4), (32, 8), (40, 2)])
def test_fp8_paged_f32_queries(dev, head_dim, per_block, hq, hkv):
    """Float32 queries over e4m3 caches, per-head or per-(page, head) scales,
    GQA, split-K lengths; float32 output."""
    lens = [0, 1, 17, 300, 1024, 1025, 3000]
    case = build_paged(lens, hq, hkv, head_dim, F32, dev, fp8=True, per_block=per_block, pool=700)
    out = cuda_llm.fp8_paged_attention_forward(case["query"], case["key_cache"],
                                               case["value_cache"], case["k_scale"],
                                               case["v_scale"], case["block_tables"],
                                               case["context_lens"])
    torch.cuda.synchronize()
    assert out.dtype == F32
    assert_close(to_np(out), paged_oracle(case, dtype=np.float64), **TOL_F32,
                 name=f"fp8 paged f32 {hq}/{hkv} per_block={per_block}")
    assert torch.all(out[0] == 0)


def test_fp8_paged_f32_nan_tail_does_not_leak(dev):
    """e4m3 NaN codes (0x7f) past a sequence's length in its last page never
    reach the output."""
    lens = [37, 5, 2100]
    case = build_paged(lens, 8, 2, 128, F32, dev, fp8=True, per_block=True)
    ref = paged_oracle(case, dtype=np.float64)
    for i, L in enumerate(lens):
        blk = int(case["block_tables"][i, (L - 1) // 16])
        case["key_cache"][blk, :, :, L % 16:] = 0x7F
        case["value_cache"][blk, :, :, L % 16:] = 0x7F
    out = cuda_llm.fp8_paged_attention_forward(case["query"], case["key_cache"],
                                               case["value_cache"], case["k_scale"],
                                               case["v_scale"], case["block_tables"],
                                               case["context_lens"])
    torch.cuda.synchronize()
    assert_close(to_np(out), ref, **TOL_F32, name="fp8 paged f32 nan tail")
