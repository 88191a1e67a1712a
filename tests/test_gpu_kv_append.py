"""GPU tier: paged KV-cache append (cuda_llm.paged_kv_append) vs the oracle.

Bit-exact against oracle.paged_append (pinned in test_oracle.py against the
reference's layout helper and quantisation recipe) for 16-bit caches, FP8
caches with per-head scales and FP8 caches with per-page scales, through
decode-style single-token appends, ragged prefill chunks that start mid-page,
invalid block ids and positions past the table; then end to end: caches built
by appends feed the paged decode kernels, checked against the oracle decode.
"""
import numpy as np
import pytest
import torch

import cuda_llm
import oracle
from _util import TOL_16BIT, TOL_FP8, assert_close, to_np

pytestmark = pytest.mark.gpu
F8 = torch.float8_e4m3fn


def _setup(dev, n=5, hkv=2, d=128, max_len=100, extra=2, seed=0):
    g = torch.Generator().manual_seed(seed)
    bps = (max_len + 15) // 16 + extra
    nblocks = n * bps + 3
    perm = torch.randperm(nblocks, generator=g)[: n * bps]
    tables = perm.view(n, bps).to(torch.int32).to(dev)
    return g, tables, nblocks


def _np_cache(c):
    return to_np(c) if c.dtype not in (torch.uint8, F8) else c.view(torch.uint8).cpu().numpy()


def _append_both(dev, key, value, kc, vc, tables, lens, new, ks=None, vs=None):
    """Run the kernel and the oracle from the same state; return both states."""
    ref = oracle.paged_append(to_np(key), to_np(value), _np_cache(kc), _np_cache(vc),
                              tables.cpu().numpy(), lens.cpu().numpy(),
                              None if new is None else new.cpu().numpy(),
                              None if ks is None else ks.cpu().numpy(),
                              None if vs is None else vs.cpu().numpy())
    cuda_llm.paged_kv_append(key, value, kc, vc, tables, lens, new, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    return ref


def _assert_state(kc, vc, ks, vs, ref):
    np.testing.assert_array_equal(_np_cache(kc), ref[0])
    np.testing.assert_array_equal(_np_cache(vc), ref[1])
    if ks is not None:
        np.testing.assert_array_equal(ks.cpu().numpy(), ref[2])
        np.testing.assert_array_equal(vs.cpu().numpy(), ref[3])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("mode", ["16bit", "fp8_head", "fp8_page"])
def test_append_sequences_of_chunks(dev, dtype, head_dim, mode):
    """A prefill chunk of ragged length, then decode steps, then another
    chunk: every call bit-exact with the oracle (whole caches compared)."""
    n, hkv = 5, 2
    g, tables, nblocks = _setup(dev, n, hkv, head_dim)
    shape = (nblocks, hkv, head_dim, 16)
    if mode == "16bit":
        kc = torch.randn(shape, generator=g).to(dtype).to(dev)
        vc = torch.randn(shape, generator=g).to(dtype).to(dev)
        ks = vs = None
    else:
        kc = torch.zeros(shape, dtype=torch.uint8, device=dev)
        vc = torch.zeros(shape, dtype=torch.uint8, device=dev)
        if mode == "fp8_head":
            ks = torch.tensor([0.01, 0.02], device=dev)
            vs = torch.tensor([0.015, 0.005], device=dev)
        else:
            ks = torch.ones(nblocks, hkv, device=dev)
            vs = torch.ones(nblocks, hkv, device=dev)
    lens = torch.zeros(n, dtype=torch.int32, device=dev)
    for step, (t, ragged) in enumerate([(37, True), (1, False), (1, True), (1, False), (21, True)]):
        key = (torch.randn(n, hkv, t, head_dim, generator=g) * (1 + step)).to(dtype).to(dev)
        value = torch.randn(n, hkv, t, head_dim, generator=g).to(dtype).to(dev)
        new = (torch.randint(0, t + 1, (n,), generator=g).to(torch.int32).to(dev) if ragged else None)
        ref = _append_both(dev, key, value, kc, vc, tables, lens, new, ks, vs)
        _assert_state(kc, vc, ks, vs, ref)
        lens += new if new is not None else t


@pytest.mark.parametrize("mode", ["16bit", "fp8_page"])
def test_append_skips_bad_blocks_and_positions(dev, mode):
    n, hkv, d = 3, 2, 64
    g, tables, nblocks = _setup(dev, n, hkv, d, max_len=40, extra=0)  # 3 pages per sequence
    tables[0, 1] = -1
    tables[1, 2] = nblocks + 7
    shape = (nblocks, hkv, d, 16)
    if mode == "16bit":
        kc = torch.randn(shape, generator=g).to(torch.bfloat16).to(dev)
        vc = torch.randn(shape, generator=g).to(torch.bfloat16).to(dev)
        ks = vs = None
    else:
        kc = torch.zeros(shape, dtype=torch.uint8, device=dev)
        vc = torch.zeros(shape, dtype=torch.uint8, device=dev)
        ks = torch.ones(nblocks, hkv, device=dev)
        vs = torch.ones(nblocks, hkv, device=dev)
    key = torch.randn(n, hkv, 30, d, generator=g).to(torch.bfloat16).to(dev)
    value = torch.randn(n, hkv, 30, d, generator=g).to(torch.bfloat16).to(dev)
    lens = torch.tensor([5, 20, 40], dtype=torch.int32, device=dev)  # the last is already full
    ref = _append_both(dev, key, value, kc, vc, tables, lens, None, ks, vs)
    _assert_state(kc, vc, ks, vs, ref)


@pytest.mark.parametrize("fp8", [False, True])
def test_appended_cache_feeds_paged_decode(dev, fp8):
    """Build every sequence's cache with a prefill chunk and decode steps, then
    run the paged decode entry point on it against the oracle decode of the
    tokens that were appended (dequantised for FP8)."""
    n, hq, hkv, d = 4, 8, 2, 128
    g, tables, nblocks = _setup(dev, n, hkv, d, max_len=300, extra=0)
    shape = (nblocks, hkv, d, 16)
    lens_final = torch.tensor([300, 1, 129, 64], dtype=torch.int32)
    tokens_k = torch.randn(n, hkv, 300, d, generator=g).to(torch.bfloat16)
    tokens_v = torch.randn(n, hkv, 300, d, generator=g).to(torch.bfloat16)
    if fp8:
        kc = torch.zeros(shape, dtype=torch.uint8, device=dev)
        vc = torch.zeros(shape, dtype=torch.uint8, device=dev)
        ks = torch.ones(nblocks, hkv, device=dev)
        vs = torch.ones(nblocks, hkv, device=dev)
    else:
        kc = torch.zeros(shape, dtype=torch.bfloat16, device=dev)
        vc = torch.zeros(shape, dtype=torch.bfloat16, device=dev)
        ks = vs = None
    lens = torch.zeros(n, dtype=torch.int32, device=dev)
    first = torch.minimum(lens_final, torch.tensor(200)).to(torch.int32)
    cuda_llm.paged_kv_append(tokens_k[:, :, :200].to(dev), tokens_v[:, :, :200].to(dev), kc, vc,
                             tables, lens, first.to(dev), k_scale=ks, v_scale=vs)
    lens += first.to(dev)
    for step in range(200, 300):
        new = (lens_final > step).to(torch.int32)
        cuda_llm.paged_kv_append(tokens_k[:, :, step:step + 1].to(dev),
                                 tokens_v[:, :, step:step + 1].to(dev), kc, vc, tables, lens,
                                 new.to(dev), k_scale=ks, v_scale=vs)
        lens += new.to(dev)
    assert torch.equal(lens.cpu(), lens_final)
    q = torch.randn(n, hq, d, generator=g).to(torch.bfloat16).to(dev)
    if fp8:
        out = cuda_llm.fp8_paged_attention_forward(q, kc, vc, ks, vs, tables, lens)
        ref = oracle.paged_decode(to_np(q), kc.cpu().numpy(), vc.cpu().numpy(),
                                  tables.cpu().numpy(), lens.cpu().numpy(),
                                  k_scale=ks.cpu().numpy(), v_scale=vs.cpu().numpy())
        tol = TOL_FP8
    else:
        out = cuda_llm.paged_attention_forward(q, kc, vc, tables, lens)
        ref = oracle.decode(to_np(q), to_np(tokens_k), to_np(tokens_v), lens_final.numpy())
        tol = TOL_16BIT
    torch.cuda.synchronize()
    assert_close(to_np(out), ref, **tol, name="decode on appended cache")
