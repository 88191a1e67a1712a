"""GPU tier: decode entry points vs the oracle.

* paged_attention_forward — the reference grid (tests/test_kernels_misc.py:26-35
  there: fp16/bf16, D in {64, 128}, context_lens [1,16,17] and [300,129,64],
  H=4), GQA, long contexts that split, zero-length sequences, NaN bytes in
  the unused tail of a page, and the BASELINE C3 shape on sampled sequences;
* fp8_paged_attention_forward — the reference's e4m3 test (xfail there,
  tests/test_kernels_misc.py:42-64; must pass here) with per-head scales, the
  per-(block, head) form, GQA, and the BASELINE C4 shape on sampled sequences;
* async_flash_decode / flash_decode — the reference grid
  (tests/test_attention.py:76-86: kv_len in {1, 63, 64, 1000}) plus GQA and
  split lengths;
* the balanced (stream-K) walk the paged kernels take for larger batches:
  ragged and empty contexts, a context cut into more partials than the merge
  loads at once (and more than 64), fewer pages than waves, GQA groups above
  16, head dim 64, both cache kinds and scale forms;
* the committed golden vectors.
"""
import os

import numpy as np
import pytest
import torch

import cuda_llm
import oracle
from _util import (TOL_16BIT, TOL_FP8, assert_close, balanced_walk_taken, build_paged,
                   paged_oracle, to_np)

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
DTYPES = [torch.float16, torch.bfloat16]


def _run_paged(case):
    if "k_scale" in case:
        return cuda_llm.fp8_paged_attention_forward(
            case["query"], case["key_cache"], case["value_cache"], case["k_scale"],
            case["v_scale"], case["block_tables"], case["context_lens"])
    return cuda_llm.paged_attention_forward(case["query"], case["key_cache"], case["value_cache"],
                                            case["block_tables"], case["context_lens"])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("context_lens", [[1, 16, 17], [300, 129, 64]])
def test_paged_attention(dev, dtype, head_dim, context_lens):
    case = build_paged(context_lens, 4, 4, head_dim, dtype, dev)
    out = _run_paged(case)
    torch.cuda.synchronize()
    assert_close(to_np(out), paged_oracle(case), **TOL_16BIT, name="paged")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("hq,hkv", [(32, 8), (8, 1), (16, 16), (40, 2)])
def test_paged_gqa_and_splits(dev, dtype, hq, hkv):
    lens = [0, 1, 15, 16, 17, 1023, 1024, 1025, 2047, 2048, 2049, 3000, 4097, 5000]
    case = build_paged(lens, hq, hkv, 128, dtype, dev, pool=2000)
    out = _run_paged(case)
    torch.cuda.synchronize()
    ref = paged_oracle(case)
    assert_close(to_np(out), ref, **TOL_16BIT, name=f"paged gqa {hq}/{hkv}")
    assert torch.all(out[0] == 0)


def test_paged_nan_tail_does_not_leak(dev):
    """Bytes past a sequence's length in its last page may be anything."""
    case = build_paged([37, 5], 8, 2, 128, torch.bfloat16, dev)
    ref = paged_oracle(case)
    for i, L in enumerate([37, 5]):
        blk = int(case["block_tables"][i, (L - 1) // 16])
        case["key_cache"][blk, :, :, L % 16:] = float("nan")
        case["value_cache"][blk, :, :, L % 16:] = float("nan")
    out = _run_paged(case)
    torch.cuda.synchronize()
    assert_close(to_np(out), ref, **TOL_16BIT, name="nan tail")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [64, 128])
def test_fp8_paged_attention_e4m3(dev, dtype, head_dim):
    """The reference's own FP8 test (per-head scales amax/448)."""
    case = build_paged([300, 129, 64], 4, 4, head_dim, dtype, dev, fp8=True, per_block=False)
    out = _run_paged(case)
    torch.cuda.synchronize()
    assert_close(to_np(out), paged_oracle(case), **TOL_FP8, name="fp8 per-head")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [64, 128])
def test_fp8_paged_per_block_gqa(dev, dtype, head_dim):
    lens = [0, 7, 16, 33, 1100, 2049, 4100]
    case = build_paged(lens, 32, 8, head_dim, dtype, dev, fp8=True, per_block=True, pool=1000)
    out = _run_paged(case)
    torch.cuda.synchronize()
    assert_close(to_np(out), paged_oracle(case), **TOL_FP8, name="fp8 per-block")


def test_fp8_cache_as_float8_dtype(dev):
    case = build_paged([100, 17], 8, 2, 128, torch.bfloat16, dev, fp8=True)
    ref = paged_oracle(case)
    case["key_cache"] = case["key_cache"].view(torch.float8_e4m3fn)
    case["value_cache"] = case["value_cache"].view(torch.float8_e4m3fn)
    out = _run_paged(case)
    torch.cuda.synchronize()
    assert_close(to_np(out), ref, **TOL_FP8, name="float8 dtype")


def _paged_value_mean(case, hq):
    """Mean of each sequence's visible V rows per query head (zeros for an
    empty context), from the paged layout [blocks, Hkv, D, page] and, for an
    FP8 cache, its e4m3 codes times their per-block or per-head scales."""
    vc = case["value_cache"]
    fp8 = "v_scale" in case
    lens = case["context_lens"].tolist()
    tables = case["block_tables"]
    hkv, d, page = vc.shape[1], vc.shape[2], vc.shape[3]
    out = torch.zeros(len(lens), hq, d, dtype=torch.float64, device=vc.device)
    for i, n in enumerate(lens):
        if n <= 0:
            continue
        t = torch.arange(n, device=vc.device)
        blk = tables[i, t // page].long()
        x = vc[blk, :, :, t % page]  # [n, Hkv, D]
        if fp8:
            x = x.view(torch.float8_e4m3fn).double()
            vs = case["v_scale"]
            x = x * (vs[blk][:, :, None] if vs.dim() == 2 else vs[None, :, None]).double()
        out[i] = x.double().mean(0).repeat_interleave(hq // hkv, dim=0)
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("fp8", [False, True])
def test_paged_zero_scale_is_value_mean(dev, dtype, fp8):
    """softmax_scale = 0: every visible token weighs the same, so each head's
    output is the mean of its sequence's V rows; a closed form that needs no
    oracle, over split-K lengths and an empty context."""
    lens = [0, 1, 17, 1030, 3000]
    case = build_paged(lens, 8, 2, 128, dtype, dev, fp8=fp8)
    args = (case["query"], case["key_cache"], case["value_cache"])
    if fp8:
        out = cuda_llm.fp8_paged_attention_forward(*args, case["k_scale"], case["v_scale"],
                                                   case["block_tables"], case["context_lens"],
                                                   softmax_scale=0.0)
    else:
        out = cuda_llm.paged_attention_forward(*args, case["block_tables"], case["context_lens"],
                                               softmax_scale=0.0)
    torch.cuda.synchronize()
    ref = _paged_value_mean(case, 8)
    tol = 1e-4 if dtype == torch.float32 else TOL_16BIT["max_abs"]
    assert (out.double() - ref).abs().max() <= tol


@pytest.mark.parametrize("fp8", [False, True])
def test_paged_zero_scale_long_context(dev, fp8):
    """A 70001-token context (4376 pages: 35 FP8 or 69 16-bit splits merged)
    beside a short one, against the closed-form value mean of softmax_scale
    = 0."""
    case = build_paged([70001, 5], 8, 2, 128, torch.bfloat16, dev, fp8=fp8)
    args = (case["query"], case["key_cache"], case["value_cache"])
    if fp8:
        out = cuda_llm.fp8_paged_attention_forward(*args, case["k_scale"], case["v_scale"],
                                                   case["block_tables"], case["context_lens"],
                                                   softmax_scale=0.0)
    else:
        out = cuda_llm.paged_attention_forward(*args, case["block_tables"], case["context_lens"],
                                               softmax_scale=0.0)
    torch.cuda.synchronize()
    ref = _paged_value_mean(case, 8)
    assert (out.double() - ref).abs().max() <= TOL_16BIT["max_abs"]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_zero_scale_is_value_mean(dev, dtype):
    q = torch.randn(2, 8, 1, 128, device=dev).to(dtype)
    k = torch.randn(2, 2, 2500, 128, device=dev).to(dtype)
    v = torch.randn(2, 2, 2500, 128, device=dev).to(dtype)
    out = cuda_llm.flash_decode(q, k, v, softmax_scale=0.0)
    torch.cuda.synchronize()
    ref = v.double().mean(2, keepdim=True).repeat_interleave(4, dim=1)
    tol = 1e-4 if dtype == torch.float32 else TOL_16BIT["max_abs"]
    assert (out.double() - ref).abs().max() <= tol


@pytest.mark.parametrize("fp8", [False, True])
def test_paged_negative_scale(dev, fp8):
    """A negative softmax_scale through the paged kernels, against the oracle."""
    case = build_paged([1, 17, 1030, 3000], 8, 2, 128, torch.bfloat16, dev, fp8=fp8)
    args = (case["query"], case["key_cache"], case["value_cache"])
    if fp8:
        out = cuda_llm.fp8_paged_attention_forward(*args, case["k_scale"], case["v_scale"],
                                                   case["block_tables"], case["context_lens"],
                                                   softmax_scale=-0.1)
    else:
        out = cuda_llm.paged_attention_forward(*args, case["block_tables"], case["context_lens"],
                                               softmax_scale=-0.1)
    torch.cuda.synchronize()
    lens = case["context_lens"].cpu().numpy()
    tables = case["block_tables"].cpu().numpy()
    if fp8:
        ref = oracle.paged_decode(to_np(case["query"]), case["key_cache"].cpu().numpy(),
                                  case["value_cache"].cpu().numpy(), tables, lens, scale=-0.1,
                                  k_scale=case["k_scale"].cpu().numpy(),
                                  v_scale=case["v_scale"].cpu().numpy())
    else:
        ref = oracle.paged_decode(to_np(case["query"]), to_np(case["key_cache"]),
                                  to_np(case["value_cache"]), tables, lens, scale=-0.1)
    assert_close(to_np(out), ref, **(TOL_FP8 if fp8 else TOL_16BIT), name=f"negative scale fp8={fp8}")


def test_golden_paged(dev):
    g = np.load(GOLDEN, allow_pickle=False)
    c = {k.split("/", 1)[1]: g[k] for k in g.files if k.startswith("paged_d64/")}
    t = lambda a, dt=None: torch.from_numpy(a).to(dev) if dt is None else torch.from_numpy(a).to(dev).to(dt)
    out = cuda_llm.paged_attention_forward(t(c["query"], torch.bfloat16), t(c["key_cache"], torch.bfloat16),
                                           t(c["value_cache"], torch.bfloat16), t(c["block_tables"]),
                                           t(c["context_lens"]))
    torch.cuda.synchronize()
    assert_close(to_np(out), c["out"], **TOL_16BIT, name="golden paged")


def test_golden_fp8_paged(dev):
    g = np.load(GOLDEN, allow_pickle=False)
    c = {k.split("/", 1)[1]: g[k] for k in g.files if k.startswith("fp8_paged_d128/")}
    t = lambda a: torch.from_numpy(a).to(dev)
    out = cuda_llm.fp8_paged_attention_forward(t(c["query"]).to(torch.bfloat16), t(c["key_cache"]),
                                               t(c["value_cache"]), t(c["k_scale"]), t(c["v_scale"]),
                                               t(c["block_tables"]), t(c["context_lens"]))
    torch.cuda.synchronize()
    assert_close(to_np(out), c["out"], **TOL_FP8, name="golden fp8 paged")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("kv_len", [1, 63, 64, 1000])
def test_decode(dev, dtype, head_dim, kv_len):
    q = torch.randn(2, 4, 1, head_dim, device=dev, dtype=dtype)
    k = torch.randn(2, 4, kv_len, head_dim, device=dev, dtype=dtype)
    v = torch.randn(2, 4, kv_len, head_dim, device=dev, dtype=dtype)
    out = cuda_llm.async_flash_decode(q, k, v)
    torch.cuda.synchronize()
    ref = oracle.attention(to_np(q), to_np(k), to_np(v))
    assert_close(to_np(out), ref, **TOL_16BIT, name="decode")


@pytest.mark.parametrize("hq,hkv,kv_len", [(32, 8, 5000), (8, 1, 1025), (4, 4, 9000)])
def test_flash_decode_gqa_split(dev, hq, hkv, kv_len):
    q = torch.randn(3, hq, 1, 128, device=dev, dtype=torch.bfloat16)
    k = torch.randn(3, hkv, kv_len, 128, device=dev, dtype=torch.bfloat16)
    v = torch.randn(3, hkv, kv_len, 128, device=dev, dtype=torch.bfloat16)
    out = cuda_llm.flash_decode(q, k, v)
    torch.cuda.synchronize()
    ref = oracle.attention(to_np(q), to_np(k), to_np(v))
    assert_close(to_np(out), ref, **TOL_16BIT, name="flash_decode gqa")


def test_baseline_c3_shape(dev):
    """C3: N=64, Hq=32/Hkv=8, D=128, L ~ U[512, 8192], 40k-page pool,
    permuted; every sequence against the oracle."""
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(512, 8193, (64,), generator=g).tolist()
    case = build_paged(lens, 32, 8, 128, torch.bfloat16, dev, pool=40000)
    out = _run_paged(case)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    ref = paged_oracle(case, list(range(64)))
    o = to_np(out)
    for n in range(64):   # every sequence, each within the 16-bit tolerance
        assert_close(o[n], ref[n], **TOL_16BIT, name=f"C3 sequence {n}")


def test_baseline_c4_shape(dev):
    """C4: N=256, L ~ U[2048, 32768], e4m3 cache with per-(page, kv-head) scales."""
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(2048, 32769, (256,), generator=g).tolist()
    case = build_paged(lens, 32, 8, 128, torch.bfloat16, dev, fp8=True, per_block=True)
    out = _run_paged(case)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    # a quarter of the sequences (every fourth, plus the longest and the
    # shortest), each within the FP8 tolerance
    seqs = sorted(set(range(0, 256, 4)) | {int(np.argmax(lens)), int(np.argmin(lens))})
    ref = paged_oracle(case, seqs)
    o = to_np(out)
    for j, n in enumerate(seqs):
        assert_close(o[n], ref[j], **TOL_FP8, name=f"C4 sequence {n}")


def _check_balanced(case, tol, fp8, name):
    n, hq, d = case["query"].shape
    hkv = case["key_cache"].shape[1]
    assert balanced_walk_taken(n, hq, hkv, d, case["block_tables"].shape[1], fp8), \
        f"{name}: these sizes do not take the balanced walk"
    out = _run_paged(case)
    again = _run_paged(case)
    torch.cuda.synchronize()
    assert torch.equal(out, again), f"{name}: not reproducible"
    ref = paged_oracle(case)
    o = to_np(out)
    for i in range(n):
        assert_close(o[i], ref[i], **tol, name=f"{name} sequence {i}")
    return out


_EDGE_LENS = [0, 1, 15, 16, 17, 1023, 1024, 1025, 2047, 2048, 2049, 4095, 4096, 4097, 8191, 8192,
              0, 0, 0, 5000]


@pytest.mark.parametrize("dtype,fp8,per_block", [(torch.bfloat16, False, True),
                                                 (torch.float16, False, True),
                                                 (torch.bfloat16, True, True),
                                                 (torch.float16, True, False)])
def test_balanced_walk_ragged(dev, dtype, fp8, per_block):
    """96 sequences, GQA 32/8: the edge lengths of a 64- / 128-page split
    (empty ones among them, written as zeros) plus random lengths up to 8192."""
    g = torch.Generator().manual_seed(11)
    lens = _EDGE_LENS + torch.randint(0, 8193, (96 - len(_EDGE_LENS),), generator=g).tolist()
    case = build_paged(lens, 32, 8, 128, dtype, dev, fp8=fp8, per_block=per_block, pool=30000,
                       seed=11)
    out = _check_balanced(case, TOL_FP8 if fp8 else TOL_16BIT, fp8, "balanced ragged")
    assert torch.all(out[0] == 0) and torch.all(out[16:19] == 0)


@pytest.mark.parametrize("fp8", [False, True])
def test_balanced_walk_long_context(dev, fp8):
    """One 65536-token context among 63 short ones: each of its kv heads is
    cut across ~100 waves, so its merge takes more partials than it loads
    ahead (16) and than one pass of lanes (64)."""
    g = torch.Generator().manual_seed(12)
    lens = [65536] + torch.randint(1, 200, (63,), generator=g).tolist()
    case = build_paged(lens, 32, 8, 128, torch.bfloat16, dev, fp8=fp8, seed=12)
    _check_balanced(case, TOL_FP8 if fp8 else TOL_16BIT, fp8, "balanced long")


def test_balanced_walk_wide_groups_and_head_dim_64(dev):
    """GQA groups of 32 query heads (two 16-head chunks per kv head) at head
    dim 128, and head dim 64."""
    g = torch.Generator().manual_seed(13)
    lens = torch.randint(0, 8193, (80,), generator=g).tolist()
    case = build_paged(lens, 64, 2, 128, torch.bfloat16, dev, pool=30000, seed=13)
    _check_balanced(case, TOL_16BIT, False, "balanced Gq=32")
    lens = torch.randint(0, 8193, (64,), generator=g).tolist()
    for fp8 in (False, True):
        case = build_paged(lens, 32, 8, 64, torch.bfloat16, dev, fp8=fp8, pool=20000, seed=14)
        _check_balanced(case, TOL_FP8 if fp8 else TOL_16BIT, fp8, f"balanced D=64 fp8={fp8}")


@pytest.mark.parametrize("n", [1024, 1025])
def test_balanced_walk_sequence_limit(dev, n):
    """1024 sequences fill every lane of the walk's prefix registers (16
    chunks of 64); 1025 exceed them and take the split grid. Short random
    contexts, a few long ones so that contexts span several splits."""
    g = torch.Generator().manual_seed(16)
    lens = torch.randint(0, 300, (n,), generator=g).tolist()
    for i in (0, 511, n - 1):
        lens[i] = 2100
    case = build_paged(lens, 32, 8, 128, torch.bfloat16, dev, seed=16)
    assert balanced_walk_taken(n, 32, 8, 128, case["block_tables"].shape[1], False) == (n <= 1024)
    out = _run_paged(case)
    torch.cuda.synchronize()
    ref = paged_oracle(case)
    assert_close(to_np(out), ref, **TOL_16BIT, name=f"N={n}")


def _widen(case, width):
    t = case["block_tables"]
    case["block_tables"] = torch.cat(
        [t, torch.zeros(t.shape[0], width - t.shape[1], dtype=t.dtype, device=t.device)], 1).contiguous()
    return case


@pytest.mark.parametrize("fp8", [False, True])
def test_balanced_walk_few_pages(dev, fp8):
    """Block tables 1024 entries wide with little context: fewer than 16
    pages per wave (the launch uses fewer waves), fewer pages than 16 in all
    (one wave), and no context at all (every row zero)."""
    cases = [[0] * 61 + [17, 3000, 9000], [0] * 63 + [5], [0] * 64]
    for lens in cases:
        case = _widen(build_paged(lens, 32, 8, 128, torch.bfloat16, dev, fp8=fp8, pool=1200,
                                  seed=15), 1024)
        out = _check_balanced(case, TOL_FP8 if fp8 else TOL_16BIT, fp8, f"few pages {lens[-3:]}")
        assert torch.all(out[:61] == 0)


@pytest.mark.parametrize("nbytes", [16, 4096 * 16 + 48, (2048 * 256 * 8 + 7) * 16])
def test_stream_read_measurement_kernel(dev, nbytes):
    """The streaming-read kernel bench.py uses as the measured HBM ceiling:
    it reads any 16-byte multiple (tails past the last full stride included)
    and leaves its input untouched."""
    import ctypes
    from cuda_amd import _lib
    x = torch.arange(nbytes // 4, dtype=torch.int32, device=dev)
    keep = x.clone()
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    _lib.call("ca_stream_read", ctypes.c_void_p(x.data_ptr()), nbytes,
              ctypes.c_void_p(sink.data_ptr()),
              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(x, keep)


def test_block_table_debug_check(dev, monkeypatch):
    """An id outside the pool in a used table entry: clamped by default (no
    error); with CUDA_LLM_CHECK_BLOCK_TABLES=1 the paged entry points raise,
    naming the entry. Unused entries past a sequence's pages are ignored."""
    case = build_paged([40, 300], 8, 2, 128, torch.bfloat16, dev, pool=64)
    nb = case["key_cache"].shape[0]
    case["block_tables"][0, 2] = nb + 5          # used: 40 tokens -> pages 0..2
    case["block_tables"][0, 10] = -7             # unused entry: never checked
    args = (case["query"], case["key_cache"], case["value_cache"], case["block_tables"],
            case["context_lens"])
    monkeypatch.delenv("CUDA_LLM_CHECK_BLOCK_TABLES", raising=False)
    out = cuda_llm.paged_attention_forward(*args)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    monkeypatch.setenv("CUDA_LLM_CHECK_BLOCK_TABLES", "1")
    with pytest.raises(RuntimeError, match=r"block_tables\[0\]\[2\]"):
        cuda_llm.paged_attention_forward(*args)
    f8 = build_paged([40, 300], 8, 2, 128, torch.bfloat16, dev, fp8=True, pool=64)
    f8["block_tables"][1, 18] = -1               # 300 tokens -> pages 0..18
    with pytest.raises(RuntimeError, match=r"block_tables\[1\]\[18\]"):
        cuda_llm.fp8_paged_attention_forward(f8["query"], f8["key_cache"], f8["value_cache"],
                                             f8["k_scale"], f8["v_scale"], f8["block_tables"],
                                             f8["context_lens"])
    case["block_tables"][0, 2] = 3               # repaired: passes the check
    cuda_llm.paged_attention_forward(*args)
