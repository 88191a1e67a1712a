"""GPU tier: prefill (flash_attention / _v3_hopper / fused_gqa) vs the oracle.

Shapes follow the reference's test grid (tests/test_attention.py:29-54 there:
fp16/bf16, D in {64, 128}, S in {64, 100, 256}, causal and not, B=2, H=4, and
the GQA (8,2), (8,8), (4,1) cases), plus the committed golden vectors and the
BASELINE C2 shapes (checked on sampled heads against the oracle and on every
head through invariants). Tolerance: max-abs 2e-2, mean-abs 2e-3 vs fp32.
"""
import os

import numpy as np
import pytest
import torch

import cuda_llm
import oracle
from _util import TOL_16BIT, assert_close, qkv, to_np

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
DTYPES = [torch.float16, torch.bfloat16]


@pytest.mark.parametrize("fn_name", ["flash_attention_forward", "flash_attention_v3_hopper"])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("seq_len", [64, 100, 256])
@pytest.mark.parametrize("is_causal", [False, True])
def test_flash_forward(dev, fn_name, dtype, head_dim, seq_len, is_causal):
    q, k, v = qkv(2, 4, seq_len, head_dim, dtype, dev)
    out = getattr(cuda_llm, fn_name)(q, k, v, is_causal=is_causal)
    torch.cuda.synchronize()
    ref = oracle.attention(to_np(q), to_np(k), to_np(v), is_causal=is_causal)
    assert_close(to_np(out), ref, **TOL_16BIT, name=fn_name)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("hq,hkv", [(8, 2), (8, 8), (4, 1)])
@pytest.mark.parametrize("is_causal", [False, True])
def test_gqa(dev, dtype, head_dim, hq, hkv, is_causal):
    q, k, v = qkv(1, hq, 100, head_dim, dtype, dev, hkv=hkv)
    out = cuda_llm.fused_gqa_forward(q, k, v, is_causal=is_causal)
    torch.cuda.synchronize()
    ref = oracle.attention(to_np(q), to_np(k), to_np(v), is_causal=is_causal)
    assert_close(to_np(out), ref, **TOL_16BIT, name="gqa")


@pytest.mark.parametrize("name", ["attn_causal_d64", "attn_full_d64", "attn_gqa_causal_d128"])
@pytest.mark.parametrize("dtype", DTYPES)
def test_golden_vectors(dev, name, dtype):
    g = np.load(GOLDEN, allow_pickle=False)
    q, k, v = (torch.from_numpy(g[f"{name}/{x}"]).to(dev).to(dtype) for x in "qkv")
    out = cuda_llm.flash_attention(q, k, v, is_causal=bool(g[f"{name}/causal"]))
    torch.cuda.synchronize()
    assert_close(to_np(out), g[f"{name}/out"], **TOL_16BIT, name=name)


@pytest.mark.parametrize("seq_len", [1, 2, 31, 129, 511])
@pytest.mark.parametrize("is_causal", [False, True])
def test_ragged_lengths(dev, seq_len, is_causal):
    q, k, v = qkv(1, 3, seq_len, 128, torch.bfloat16, dev)
    out = cuda_llm.flash_attention(q, k, v, is_causal=is_causal)
    torch.cuda.synchronize()
    ref = oracle.attention(to_np(q), to_np(k), to_np(v), is_causal=is_causal)
    assert_close(to_np(out), ref, **TOL_16BIT, name=f"S={seq_len}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("is_causal", [False, True])
def test_zero_scale_is_running_mean(dev, dtype, head_dim, is_causal):
    """softmax_scale = 0 weighs every visible key equally: row i is the mean
    of V over keys 0..i (causal) or over all keys, a closed form that needs
    no oracle. Every weight is exactly 1 in the P operand, so only the fp32
    sums and the output rounding separate the kernels from it; 8 x 8 heads
    of 2100 rows give the persistent launch several items per workgroup."""
    q, k, v = qkv(8, 8, 2100, head_dim, dtype, dev)
    out = cuda_llm.flash_attention(q, k, v, is_causal=is_causal, softmax_scale=0.0)
    torch.cuda.synchronize()
    v64 = v.double()
    s = v.shape[2]
    if is_causal:
        ref = v64.cumsum(2) / torch.arange(1, s + 1, device=dev, dtype=torch.float64)[:, None]
    else:
        ref = v64.mean(2, keepdim=True).expand_as(v64)
    assert_close(to_np(out), ref.cpu().numpy(), **TOL_16BIT, name=f"zero scale {dtype}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("is_causal", [False, True])
def test_long_ragged_sequence_zero_scale(dev, dtype, head_dim, is_causal):
    """One head of 65573 rows (a ragged end far past the sizes the oracle
    checks; 1025 key tiles, so the head-dim-64 walk's groups of four end
    mid-group): with softmax_scale = 0 the output is the running mean of V,
    checked on every row."""
    s = 65573
    q, k, v = qkv(1, 1, s, head_dim, dtype, dev)
    out = cuda_llm.flash_attention(q, k, v, is_causal=is_causal, softmax_scale=0.0)
    torch.cuda.synchronize()
    v64 = v.double()
    if is_causal:
        ref = v64.cumsum(2) / torch.arange(1, s + 1, device=dev, dtype=torch.float64)[:, None]
    else:
        ref = v64.mean(2, keepdim=True).expand_as(v64)
    tol = 1e-4 if dtype == torch.float32 else TOL_16BIT["max_abs"]
    assert (out.double() - ref).abs().max().item() <= tol


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("is_causal", [False, True])
def test_negative_scale(dev, dtype, head_dim, is_causal):
    """A negative softmax_scale (the kernels' second instantiation, which
    tracks a running minimum of the raw logits) against the oracle, over
    ragged and multi-tile walks."""
    q, k, v = qkv(2, 4, 777, head_dim, dtype, dev)
    out = cuda_llm.flash_attention(q, k, v, is_causal=is_causal, softmax_scale=-0.15)
    torch.cuda.synchronize()
    ref = oracle.attention(to_np(q), to_np(k), to_np(v), is_causal=is_causal, scale=-0.15)
    assert_close(to_np(out), ref, **TOL_16BIT, name=f"negative scale {dtype}")


def test_custom_scale_and_large_logits(dev):
    """Scaled-up queries drive the lazy-rescale path (row max jumps by > 8 in
    log2 units between tiles)."""
    q, k, v = qkv(1, 2, 700, 128, torch.bfloat16, dev)
    q = (q.float() * 6).to(torch.bfloat16)
    for causal in (False, True):
        out = cuda_llm.flash_attention(q, k, v, is_causal=causal, softmax_scale=0.3)
        torch.cuda.synchronize()
        ref = oracle.attention(to_np(q), to_np(k), to_np(v), is_causal=causal, scale=0.3)
        assert_close(to_np(out), ref, **TOL_16BIT, name=f"large logits causal={causal}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("profile", ["ramp", "jump"])
@pytest.mark.parametrize("d", [64, 128])
def test_running_max_growth(dev, dtype, is_causal, profile, d):
    """Logits that grow along the keys. Tiles after a wave's first take their
    exponentials against the running max as it stands; a tile whose sums
    pass the bound of the P operand type (bf16 2^48, fp16 2^15; ramp: about
    +33 log2 units per 64-key tile) or overflow to infinity (jump: +130 log2
    units at key 512) takes the full max, rescales O and l, and takes the
    exponentials again."""
    g = torch.Generator(device=dev).manual_seed(11)
    b, h, s = 1, 2, 1024
    u = torch.randn(d, device=dev, generator=g)
    u = u / u.norm()
    j = torch.arange(s, device=dev, dtype=torch.float32)
    amp = 0.5 * j if profile == "ramp" else torch.where(j < 512, torch.ones_like(j),
                                                         torch.full_like(j, 130.0))
    k = (amp[:, None] * u + 0.1 * torch.randn(b, h, s, d, device=dev, generator=g)).to(dtype)
    q = (8 * u + 0.1 * torch.randn(b, h, s, d, device=dev, generator=g)).to(dtype)
    v = torch.randn(b, h, s, d, device=dev, generator=g).to(dtype)
    out = cuda_llm.flash_attention(q, k, v, is_causal=is_causal)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    ref = oracle.attention(to_np(q), to_np(k), to_np(v), is_causal=is_causal)
    assert_close(to_np(out), ref, **TOL_16BIT, name=f"{profile} causal={is_causal}")


def test_every_row_written(dev):
    """Output pre-filled with NaN through the C ABI: every row must be written."""
    import cuda_amd._lib as L
    from cuda_amd.api import _ptr, _stream
    q, k, v = qkv(2, 4, 333, 64, torch.bfloat16, dev)
    out = torch.full_like(q, float("nan"))
    L.call("ca_flash_attention_fwd", L.CA_BF16, _ptr(q), _ptr(k), _ptr(v), _ptr(out), 2, 4, 4,
           333, 64, 0.125, 1, _stream())
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()


def test_runs_on_current_stream(dev):
    """Calls enqueue on torch's current stream (a side stream here), as the
    reference's binding does with getCurrentCUDAStream."""
    from cuda_amd.api import _stream
    q, k, v = qkv(2, 4, 300, 128, torch.bfloat16, dev)
    ref = cuda_llm.flash_attention(q, k, v, is_causal=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert (_stream().value or 0) == side.cuda_stream
        out = cuda_llm.flash_attention(q, k, v, is_causal=True)
    assert (_stream().value or 0) == torch.cuda.current_stream().cuda_stream  # NULL = default
    side.synchronize()
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_deterministic(dev):
    q, k, v = qkv(2, 8, 1000, 128, torch.bfloat16, dev)
    a = cuda_llm.flash_attention(q, k, v, is_causal=True)
    b = cuda_llm.flash_attention(q, k, v, is_causal=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("cfg", [
    dict(b=4, h=32, s=4096, causal=True),
    dict(b=4, h=32, s=2048, causal=False),
])
def test_baseline_c2_shapes(dev, cfg):
    """BASELINE C2 (bf16 prefill B=4, H=32, S=4096 causal / 2048 non-causal,
    D=128): every head against the oracle, each head within the 16-bit
    tolerance."""
    b, h, s = cfg["b"], cfg["h"], cfg["s"]
    q, k, v = qkv(b, h, s, 128, torch.bfloat16, dev)
    out = cuda_llm.flash_attention(q, k, v, is_causal=cfg["causal"])
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    ref = oracle.attention(to_np(q), to_np(k), to_np(v), is_causal=cfg["causal"])
    o = to_np(out)
    for bi in range(b):
        for hi in range(h):
            assert_close(o[bi, hi], ref[bi, hi], **TOL_16BIT, name=f"head {bi},{hi}")
    if cfg["causal"]:
        # row 0 attends only to key 0: output equals v[..., 0, :] up to bf16 rounding
        assert (out[:, :, 0].float() - v[:, :, 0].float()).abs().max().item() <= 1e-2


@pytest.mark.parametrize("dtype,d,b,hq,hkv,s", [
    (torch.bfloat16, 128, 2, 32, 8, 3072),   # 12 query tiles of 256 rows: 6 pairs per head
    (torch.float16, 128, 2, 32, 32, 3456),   # 14 tiles (first one 128 rows): 7 pairs
    (torch.bfloat16, 128, 2, 32, 8, 3800),   # 15 tiles: 7 pairs + middle tiles of 2 heads
    (torch.float16, 128, 2, 32, 32, 4096),   # 16 tiles: 8 pairs
    (torch.bfloat16, 128, 7, 7, 1, 2800),    # 11 tiles, 49 heads: one lone middle tile
    (torch.bfloat16, 64, 4, 32, 8, 1900),    # head dim 64: 8 tiles (first one 128 rows)
    (torch.bfloat16, 128, 2, 24, 8, 3640),   # 15 tiles, the first one 64 rows (one key tile)
    (torch.float16, 64, 2, 24, 8, 3640),     # the same at head dim 64
])
def test_causal_paired_query_tiles(dev, dtype, d, b, hq, hkv, s):
    """Causal grids big enough that each workgroup takes two query tiles
    (tiles n_qt-1-p and p of a head; for an odd n_qt the middle tiles of two
    heads), for equal work per workgroup on a 256-CU device; every grid here
    also exceeds 256 such items, so each workgroup of the persistent launch
    takes several, its key ring running on from one tile into the next (a
    one-key-tile first tile, S = 3640, stops that). Sampled heads (including
    the last head, whose middle tile may be alone) against the oracle, every
    head through row 0 (which sees key 0 only) and through finiteness."""
    q, k, v = qkv(b, hq, s, d, dtype, dev, hkv=hkv)
    out = cuda_llm.flash_attention(q, k, v, is_causal=True)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    for (bi, hi) in [(0, 0), (b - 1, hq // 2 + 1), (b - 1, hq - 1)]:
        kh = hi // (hq // hkv)
        ref = oracle.attention(to_np(q[bi:bi + 1, hi:hi + 1]), to_np(k[bi:bi + 1, kh:kh + 1]),
                               to_np(v[bi:bi + 1, kh:kh + 1]), is_causal=True)
        assert_close(to_np(out[bi:bi + 1, hi:hi + 1]), ref, **TOL_16BIT, name=f"head {bi},{hi}")
    kv0 = v[:, :, 0].float().repeat_interleave(hq // hkv, dim=1)
    assert (out[:, :, 0].float() - kv0).abs().max().item() <= 1e-2


@pytest.mark.parametrize("dtype,s,d", [(torch.bfloat16, 1536, 128), (torch.bfloat16, 4096, 128),
                                       (torch.bfloat16, 3640, 128), (torch.bfloat16, 3640, 64),
                                       (torch.float16, 4096, 128), (torch.float16, 3640, 128)])
def test_persistent_noncausal(dev, dtype, s, d):
    """Non-causal grids of more than 256 query tiles: the persistent launch,
    whose workgroups take several tiles each, the key ring running on from
    one tile into the next; S = 3640 is ragged (the first tile holds 64 rows).
    fp16 at head dim 128 runs the same 64-row kernel as bf16."""
    b, hq, hkv = (4, 32, 8) if s == 1536 else (2, 32, 8)
    q, k, v = qkv(b, hq, s, d, dtype, dev, hkv=hkv)
    out = cuda_llm.flash_attention(q, k, v, is_causal=False)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    for (bi, hi) in [(0, 0), (b - 1, 13), (b - 1, hq - 1)]:
        kh = hi // (hq // hkv)
        ref = oracle.attention(to_np(q[bi:bi + 1, hi:hi + 1]), to_np(k[bi:bi + 1, kh:kh + 1]),
                               to_np(v[bi:bi + 1, kh:kh + 1]))
        assert_close(to_np(out[bi:bi + 1, hi:hi + 1]), ref, **TOL_16BIT, name=f"head {bi},{hi}")


def _random_w64_cases(n=12, seed=1234):
    """Seeded shapes for the 64-row kernel (head dim 128, bf16 and fp16):
    ragged lengths (a first query tile of 64-192 rows), GQA ratios, causal
    and not, with and without the LSE output."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        hkv = int(rng.choice([1, 2, 4, 8]))
        g = int(rng.choice([1, 2, 4]))
        s = int(rng.integers(65, 2600))
        out.append((torch.float16 if i % 2 else torch.bfloat16, int(rng.integers(1, 3)), hkv * g, hkv, s,
                    bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), float(rng.choice([0.05, 0.0884, 0.2]))))
    return out


@pytest.mark.parametrize("dtype,b,hq,hkv,s,causal,lse,scale", _random_w64_cases())
def test_w64_random_shapes(dev, dtype, b, hq, hkv, s, causal, lse, scale):
    """The 64-row kernel on seeded random shapes: every head of the first
    batch against the oracle; the LSE, where asked for, against the oracle's
    logsumexp."""
    gen = torch.Generator(device=dev).manual_seed(s)
    q, k, v = qkv(b, hq, s, 128, dtype, dev, hkv=hkv, gen=gen)
    if lse:
        out, l = cuda_llm.flash_attention_forward_lse(q, k, v, is_causal=causal, softmax_scale=scale)
    else:
        out = cuda_llm.flash_attention(q, k, v, is_causal=causal, softmax_scale=scale)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    ref = oracle.attention(to_np(q[:1]), to_np(k[:1]), to_np(v[:1]), is_causal=causal, scale=scale)
    assert_close(to_np(out[:1]), ref, **TOL_16BIT, name=f"{dtype} {b}x{hq}/{hkv}x{s} causal={causal}")
    if lse:
        lref = oracle.attention_lse(to_np(q[:1]), to_np(k[:1]), is_causal=causal, scale=scale, dtype=np.float64)
        assert np.abs(to_np(l[:1]) - lref).max() <= 1e-3


@pytest.mark.parametrize("dtype,s,causal", [(torch.bfloat16, 16384, True), (torch.float16, 16384, False),
                                            (torch.bfloat16, 12345, False)])
def test_w64_long_sequences(dev, dtype, s, causal):
    """Long walks of the 64-row kernel (up to 256 key tiles per query tile,
    64 query tiles per head) on one head against the oracle."""
    gen = torch.Generator(device=dev).manual_seed(s)
    q, k, v = qkv(1, 2, s, 128, dtype, dev, gen=gen)
    out = cuda_llm.flash_attention(q, k, v, is_causal=causal)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    ref = oracle.attention(to_np(q[:, 1:]), to_np(k[:, 1:]), to_np(v[:, 1:]), is_causal=causal)
    assert_close(to_np(out[:, 1:]), ref, **TOL_16BIT, name=f"{dtype} S={s} causal={causal}")
