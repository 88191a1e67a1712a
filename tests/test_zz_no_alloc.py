"""GPU tier: ca_fp8_paged_attention_noalloc, the FP8 paged decode entry point
that allocates nothing (split-K partials in the library's per-device scratch).

Called through the C ABI and compared with ca_fp8_paged_attention (the
workspace form, same kernels) bit for bit, on two calls in a row whose second
is smaller (the scratch keeps the first call's partials), and with the oracle
at the FP8 tolerance. No counterpart in the reference.
"""
import ctypes

import numpy as np
import pytest
import torch

import cuda_amd._lib as L
import cuda_llm
from _util import TOL_FP8, assert_close, balanced_walk_taken, build_paged, paged_oracle, to_np

pytestmark = pytest.mark.gpu


def _noalloc(case, scale=None, stream=None):
    q = case["query"]
    n, hq, d = q.shape
    kc = case["key_cache"]
    per_block = case["k_scale"].dim() == 2
    out = torch.empty_like(q)
    dt = {torch.bfloat16: L.CA_BF16, torch.float16: L.CA_F16, torch.float32: L.CA_F32}[q.dtype]
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    L.call("ca_fp8_paged_attention_noalloc", dt, p(q), p(kc), p(case["value_cache"]),
           p(case["k_scale"]), p(case["v_scale"]), int(per_block), p(case["block_tables"]),
           p(case["context_lens"]), p(out), n, hq, kc.shape[1], d, case["block_tables"].shape[1],
           16, kc.shape[0], 1.0 / d ** 0.5 if scale is None else scale,
           ctypes.c_void_p((stream or torch.cuda.current_stream()).cuda_stream))
    return out


def _with_workspace(case):
    return cuda_llm.fp8_paged_attention_forward(case["query"], case["key_cache"],
                                                case["value_cache"], case["k_scale"],
                                                case["v_scale"], case["block_tables"],
                                                case["context_lens"])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_form_twice(dev, dtype):
    # first call: 4 sequences, up to 5000 tokens (3 splits of 128 pages), GQA 32/8
    big = build_paged([5000, 3000, 200, 0], 32, 8, 128, dtype, dev, fp8=True, per_block=True,
                      pool=700, seed=1)
    # second call: smaller (2 sequences, 2 splits, per-head scales), other data
    small = build_paged([2100, 17], 8, 2, 128, dtype, dev, fp8=True, per_block=False, seed=2)
    for case, name in ((big, "first"), (small, "second, smaller")):
        out = _noalloc(case)
        ref = _with_workspace(case)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"{name}: differs from ca_fp8_paged_attention"
        tol = TOL_FP8 if dtype != torch.float32 else dict(max_abs=1e-4, mean_abs=1e-5)
        assert_close(to_np(out), paged_oracle(case, dtype=np.float64), **tol, name=name)
    assert torch.all(_noalloc(big)[3] == 0)  # empty context -> zero row


def test_noalloc_balanced_walk_twice(dev):
    """Sizes that take the balanced (stream-K) walk, whose partials and
    per-sequence prefix also live in the scratch: two calls in a row, the
    second smaller, each bit for bit the workspace form's and within the FP8
    tolerance of the oracle."""
    g = torch.Generator().manual_seed(5)
    big = build_paged(torch.randint(0, 16385, (100,), generator=g).tolist(), 32, 8, 128,
                      torch.bfloat16, dev, fp8=True, per_block=True, seed=5)
    small = build_paged(torch.randint(0, 8193, (64,), generator=g).tolist(), 32, 8, 128,
                        torch.bfloat16, dev, fp8=True, per_block=False, seed=6)
    for case, name in ((big, "first"), (small, "second, smaller")):
        n, hq, d = case["query"].shape
        assert balanced_walk_taken(n, hq, 8, d, case["block_tables"].shape[1], True), name
        out = _noalloc(case)
        ref = _with_workspace(case)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"{name}: differs from ca_fp8_paged_attention"
        assert_close(to_np(out), paged_oracle(case, dtype=np.float64), **TOL_FP8, name=name)


def test_noalloc_serves_c4(dev):
    """At the C4 shape (256 sequences up to 32768 tokens, GQA 32/8) the
    balanced walk's partials fit the scratch: the allocation-free form runs
    it and equals the workspace form bit for bit."""
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(2048, 32769, (256,), generator=g).tolist()
    case = build_paged(lens, 32, 8, 128, torch.bfloat16, dev, fp8=True, per_block=True)
    assert balanced_walk_taken(256, 32, 8, 128, case["block_tables"].shape[1], True)
    out = _noalloc(case)
    ref = _with_workspace(case)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert torch.equal(out, ref)


def test_noalloc_two_streams(dev):
    """Calls on two streams, issued back to back with no host wait between,
    share the scratch: the second call's stream waits for the first call on
    the GPU, so both outputs equal the workspace form bit for bit."""
    big = build_paged([5000, 4000, 3000, 2600], 32, 8, 128, torch.bfloat16, dev, fp8=True,
                      per_block=True, pool=1200, seed=3)
    small = build_paged([2100, 2000, 1900], 32, 8, 128, torch.bfloat16, dev, fp8=True,
                        per_block=True, pool=400, seed=4)
    refs = [_with_workspace(c) for c in (big, small)]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for _ in range(3):
        a = _noalloc(big, stream=s1)
        b = _noalloc(small, stream=s2)
        c = _noalloc(big, stream=s1)
        torch.cuda.synchronize()
        assert torch.equal(a, refs[0]) and torch.equal(b, refs[1]) and torch.equal(c, refs[0])


def test_noalloc_rejects_sizes_beyond_scratch(dev):
    case = build_paged([16], 32, 8, 128, torch.bfloat16, dev, fp8=True, per_block=True)
    # 1100 sequences (more than the balanced walk's 1024, so the split grid)
    # with a table 2048 blocks wide need 1100*32*16*129*4 bytes of partials
    q = torch.zeros(1100, 32, 128, dtype=torch.bfloat16, device=dev)
    tables = torch.zeros(1100, 2048, dtype=torch.int32, device=dev)
    lens = torch.zeros(1100, dtype=torch.int32, device=dev)
    big = dict(case, query=q, block_tables=tables, context_lens=lens)
    with pytest.raises(RuntimeError, match="scratch"):
        _noalloc(big)
