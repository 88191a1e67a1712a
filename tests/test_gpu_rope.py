"""GPU tier: fused_rope_flash_attention vs the oracle.

The reference's test (tests/test_attention.py:57-70 there): fp16 / bf16, head
dims 64 and 128, S = 100, B = 1, H = 4, causal and not, tables from
rope_tables (tests/_utils.py:75-81), against ref_rope_attention. Here the same
grid plus float32, GQA and longer S, and the identity tables (cos = 1,
sin = 0), which must reproduce flash_attention bit for bit.
"""
import numpy as np
import pytest
import torch

import cuda_llm
import oracle
from _util import TOL_16BIT, assert_close, qkv, to_np

pytestmark = pytest.mark.gpu
TOL_F32 = dict(max_abs=1e-4, mean_abs=1e-5)


def rope_tables(s, d, dev, base=10000.0):
    """tests/_utils.py:75-81: cos / sin [S, D], rotate-half convention."""
    inv = 1.0 / (base ** (torch.arange(0, d, 2, device=dev).float() / d))
    t = torch.arange(s, device=dev, dtype=torch.float32)
    emb = torch.cat([torch.outer(t, inv)] * 2, dim=-1)
    return emb.cos().contiguous(), emb.sin().contiguous()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("is_causal", [False, True])
def test_rope_reference_grid(dev, dtype, head_dim, is_causal):
    q, k, v = qkv(1, 4, 100, head_dim, dtype, dev)
    cos, sin = rope_tables(100, head_dim, dev)
    out = cuda_llm.fused_rope_flash_attention(q, k, v, cos, sin, is_causal=is_causal)
    torch.cuda.synchronize()
    ref = oracle.rope_attention(to_np(q), to_np(k), to_np(v), to_np(cos), to_np(sin),
                                is_causal=is_causal, dtype=np.float64)
    tol = TOL_F32 if dtype == torch.float32 else TOL_16BIT
    assert_close(to_np(out), ref, **tol, name="rope")


@pytest.mark.parametrize("b,hq,hkv,s,d", [(2, 8, 2, 1024, 128), (1, 4, 4, 777, 64), (2, 32, 8, 2048, 128),
                                           (2, 32, 8, 4096, 128)])
def test_rope_longer_and_gqa(dev, b, hq, hkv, s, d):
    """Longer sequences and GQA; at S = 4096 the grid is persistent (512
    causal pairs), so the rotated Q of a query tile is often loaded by the
    workgroup's previous tile, of another head."""
    q, k, v = qkv(b, hq, s, d, torch.bfloat16, dev, hkv=hkv)
    cos, sin = rope_tables(s, d, dev)
    out = cuda_llm.fused_rope_flash_attention(q, k, v, cos, sin)  # default causal
    torch.cuda.synchronize()
    for (bi, hi) in [(0, 0), (b - 1, hq - 1)]:
        kh = hi // (hq // hkv)
        ref = oracle.rope_attention(to_np(q[bi:bi + 1, hi:hi + 1]), to_np(k[bi:bi + 1, kh:kh + 1]),
                                    to_np(v[bi:bi + 1, kh:kh + 1]), to_np(cos), to_np(sin),
                                    is_causal=True)
        assert_close(to_np(out[bi:bi + 1, hi:hi + 1]), ref, **TOL_16BIT, name=f"head {bi},{hi}")


@pytest.mark.parametrize("dtype,d", [(torch.float16, 128), (torch.bfloat16, 64), (torch.bfloat16, 128)])
def test_rope_identity_tables_equal_flash_attention(dev, dtype, d):
    """Identity tables leave Q and K as they are. Where both calls run the
    same kernel the outputs are equal bit for bit; at head dim 128 without
    rope both 16-bit types run the 64-row kernel, whose summation order
    differs, so there the two agree to the 16-bit tolerance."""
    q, k, v = qkv(2, 4, 300, d, dtype, dev)
    ones = torch.ones(300, d, device=dev)
    zeros = torch.zeros(300, d, device=dev)
    a = cuda_llm.fused_rope_flash_attention(q, k, v, ones, zeros, is_causal=True)
    b = cuda_llm.flash_attention(q, k, v, is_causal=True)
    torch.cuda.synchronize()
    if d == 128:
        assert_close(to_np(a), to_np(b), **TOL_16BIT, name="identity rope")
    else:
        assert torch.equal(a, b)


def test_rope_rejects_bad_tables(dev):
    q, k, v = qkv(1, 2, 64, 64, torch.bfloat16, dev)
    cos, sin = rope_tables(32, 64, dev)
    with pytest.raises(RuntimeError, match="seq_len, head_dim"):
        cuda_llm.fused_rope_flash_attention(q, k, v, cos, sin)
