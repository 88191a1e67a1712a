"""GPU tier: flash-attention backward and the forward's LSE vs the oracle.

The reference's backward test (tests/test_attention.py:111-132 there): fp16 /
bf16, head_dim 64, S in {64, 100}, causal and not, B = 1, H = 2; out and lse
from the fp32 math; tolerance atol = rtol = 5e-2 on dq, dk, dv against fp32
autograd. Here the same grid (plus head_dim 128), larger and ragged S, GQA,
a custom scale, the forward's LSE, autograd through cuda_llm.flash_attention
and determinism; the oracle (oracle.attention_backward, pinned against torch
fp64 autograd and finite differences) runs in float64 on the same rounded
inputs. Tolerance: |err| <= 5e-2 + 5e-2 |ref| (the reference's), and a mean
absolute error below 5e-3.
"""
import numpy as np
import pytest
import torch

import cuda_llm
import oracle
from _util import qkv, to_np

pytestmark = pytest.mark.gpu
DTYPES = [torch.float16, torch.bfloat16]


def _check_grad(out, ref, name, atol=5e-2, rtol=5e-2, mean_abs=5e-3):
    out = to_np(out).astype(np.float64)
    assert out.shape == ref.shape, f"{name}: shape {out.shape} != {ref.shape}"
    assert np.isfinite(out).all(), f"{name}: non-finite values"
    err = np.abs(out - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), f"{name}: {bad.sum()} elements out of tolerance, max abs err {err.max():.3e}"
    assert err.mean() <= mean_abs, f"{name}: mean abs error {err.mean():.3e} > {mean_abs}"


def _run_backward(b, hq, hkv, s, d, dtype, dev, is_causal, scale=None, seed=0):
    """out and lse from the float64 oracle forward (out rounded to the dtype,
    as the reference test does); gradients from the kernel and from the
    oracle on the same rounded q, k, v, out, dout."""
    g = torch.Generator(device=dev).manual_seed(seed)
    q, k, v = qkv(b, hq, s, d, dtype, dev, hkv=hkv, gen=g)
    dout = torch.randn(b, hq, s, d, device=dev, generator=g).to(dtype)
    qn, kn, vn, dn = (to_np(t).astype(np.float64) for t in (q, k, v, dout))
    o = oracle.attention(qn, kn, vn, is_causal=is_causal, scale=scale, dtype=np.float64)
    lse = oracle.attention_lse(qn, kn, is_causal=is_causal, scale=scale, dtype=np.float64)
    out = torch.from_numpy(o).to(dev).to(dtype)
    dq, dk, dv = cuda_llm.flash_attention_backward(dout, q, k, v, out,
                                                   torch.from_numpy(lse).to(dev).float(),
                                                   is_causal=is_causal, softmax_scale=scale)
    torch.cuda.synchronize()
    ref = oracle.attention_backward(dn, qn, kn, vn, to_np(out).astype(np.float64), lse,
                                    is_causal=is_causal, scale=scale, dtype=np.float64)
    return (dq, dk, dv), ref


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("seq_len", [64, 100])
@pytest.mark.parametrize("is_causal", [False, True])
def test_backward_reference_grid(dev, dtype, head_dim, seq_len, is_causal):
    got, ref = _run_backward(1, 2, 2, seq_len, head_dim, dtype, dev, is_causal)
    for name, a, r in zip(("dq", "dk", "dv"), got, ref):
        _check_grad(a, r, name)


@pytest.mark.parametrize("b,hq,hkv,s,d", [
    (2, 4, 4, 1, 64), (2, 4, 4, 257, 128), (1, 8, 2, 300, 128), (1, 4, 1, 1024, 64),
    (2, 2, 2, 640, 128),
])
@pytest.mark.parametrize("is_causal", [False, True])
def test_backward_shapes_and_gqa(dev, b, hq, hkv, s, d, is_causal):
    got, ref = _run_backward(b, hq, hkv, s, d, torch.bfloat16, dev, is_causal, seed=1)
    for name, a, r in zip(("dq", "dk", "dv"), got, ref):
        _check_grad(a, r, f"{name} {b},{hq},{hkv},{s},{d}")


def test_backward_custom_scale(dev):
    got, ref = _run_backward(1, 2, 2, 200, 128, torch.float16, dev, True, scale=0.3, seed=2)
    for name, a, r in zip(("dq", "dk", "dv"), got, ref):
        _check_grad(a, r, name)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("hq,hkv,s", [(4, 4, 1), (4, 4, 50), (4, 4, 100), (8, 2, 777), (4, 4, 4096)])
@pytest.mark.parametrize("is_causal", [False, True])
def test_forward_lse(dev, dtype, head_dim, hq, hkv, s, is_causal):
    """Also one-tile walks (s <= 64), whose row max is taken in the same
    iteration as the exponentials."""
    q, k, v = qkv(1, hq, s, head_dim, dtype, dev, hkv=hkv)
    out, lse = cuda_llm.flash_attention_forward_lse(q, k, v, is_causal=is_causal)
    torch.cuda.synchronize()
    assert lse.dtype == torch.float32 and lse.shape == (1, hq, s)
    ref = oracle.attention_lse(to_np(q), to_np(k), is_causal=is_causal, dtype=np.float64)
    assert np.abs(to_np(lse) - ref).max() <= 1e-3
    plain = cuda_llm.flash_attention_forward(q, k, v, is_causal=is_causal)
    assert torch.equal(out, plain)  # the LSE store does not change O


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("is_causal", [False, True])
def test_zero_scale_closed_forms(dev, dtype, head_dim, is_causal):
    """softmax_scale = 0, end to end through the kernels' own forward (with
    LSE) and backward, against closed forms that need no oracle: P[i, j] =
    1 / n_i over the n_i visible keys of row i, so O = that running mean of
    V, LSE = ln n_i, dV = P^T dO, and dQ = dK = 0 (every logit gradient is
    multiplied by the scale)."""
    s = 300
    q, k, v = qkv(1, 2, s, head_dim, dtype, dev)
    dout = torch.randn(1, 2, s, head_dim, device=dev).to(dtype)
    out, lse = cuda_llm.flash_attention_forward_lse(q, k, v, is_causal=is_causal, softmax_scale=0.0)
    dq, dk, dv = cuda_llm.flash_attention_backward(dout, q, k, v, out, lse, is_causal=is_causal,
                                                   softmax_scale=0.0)
    torch.cuda.synchronize()
    n = torch.arange(1, s + 1, device=dev, dtype=torch.float64) if is_causal else \
        torch.full((s,), float(s), device=dev, dtype=torch.float64)
    p = (torch.tril(torch.ones(s, s, device=dev, dtype=torch.float64)) if is_causal else
         torch.ones(s, s, device=dev, dtype=torch.float64)) / n[:, None]
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert (out.double() - p @ v.double()).abs().max() <= tol
    assert (lse.double() - torch.log(n)).abs().max() <= 1e-4
    assert (dv.double() - p.t() @ dout.double()).abs().max() <= (1e-3 if dtype == torch.float32 else 5e-2)
    assert torch.count_nonzero(dq) == 0 and torch.count_nonzero(dk) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("is_causal", [False, True])
def test_zero_scale_long_ragged(dev, dtype, is_causal):
    """The zero-scale closed forms at a ragged length of 8197 rows, far past
    the sizes the oracle checks, without forming P: O is the running mean of
    V, LSE = ln n_i, dV[j] = sum over the rows i that see key j of
    dO[i] / n_i (a reversed cumulative sum when causal), dQ = dK = 0."""
    s, d = 8197, 128
    q, k, v = qkv(1, 1, s, d, dtype, dev)
    dout = torch.randn(1, 1, s, d, device=dev).to(dtype)
    out, lse = cuda_llm.flash_attention_forward_lse(q, k, v, is_causal=is_causal, softmax_scale=0.0)
    dq, dk, dv = cuda_llm.flash_attention_backward(dout, q, k, v, out, lse, is_causal=is_causal,
                                                   softmax_scale=0.0)
    torch.cuda.synchronize()
    v64, g64 = v.double()[0, 0], dout.double()[0, 0]
    if is_causal:
        n = torch.arange(1, s + 1, device=dev, dtype=torch.float64)
        o_ref = v64.cumsum(0) / n[:, None]
        dv_ref = (g64 / n[:, None]).flip(0).cumsum(0).flip(0)
    else:
        n = torch.full((s,), float(s), device=dev, dtype=torch.float64)
        o_ref = v64.mean(0, keepdim=True).expand(s, d)
        dv_ref = g64.sum(0, keepdim=True).expand(s, d) / s
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert (out.double()[0, 0] - o_ref).abs().max() <= tol
    assert (lse.double()[0, 0] - torch.log(n)).abs().max() <= 1e-4
    assert (dv.double()[0, 0] - dv_ref).abs().max() <= (1e-3 if dtype == torch.float32 else 5e-2)
    assert torch.count_nonzero(dq) == 0 and torch.count_nonzero(dk) == 0


def test_forward_lse_float32(dev):
    q, k, v = qkv(2, 4, 300, 128, torch.float32, dev)
    _, lse = cuda_llm.flash_attention_forward_lse(q, k, v, is_causal=True)
    torch.cuda.synchronize()
    ref = oracle.attention_lse(to_np(q), to_np(k), is_causal=True, dtype=np.float64)
    assert np.abs(to_np(lse) - ref).max() <= 1e-4


@pytest.mark.parametrize("is_causal", [False, True])
def test_autograd_through_flash_attention(dev, is_causal):
    """README.md:66-71: out = cllm.flash_attention(q, k, v); out.backward()."""
    q, k, v = qkv(2, 4, 300, 64, torch.bfloat16, dev)
    q, k, v = (t.requires_grad_() for t in (q, k, v))
    out = cuda_llm.flash_attention(q, k, v, is_causal=is_causal)
    dout = torch.randn_like(out)
    out.backward(dout)
    torch.cuda.synchronize()
    qn, kn, vn, dn = (to_np(t.detach()).astype(np.float64) for t in (q, k, v, dout))
    on = to_np(out.detach()).astype(np.float64)
    lse = oracle.attention_lse(qn, kn, is_causal=is_causal, dtype=np.float64)
    rq, rk, rv = oracle.attention_backward(dn, qn, kn, vn, on, lse, is_causal=is_causal,
                                           dtype=np.float64)
    for name, a, r in zip(("dq", "dk", "dv"), (q.grad, k.grad, v.grad), (rq, rk, rv)):
        _check_grad(a, r, name)


def test_autograd_gqa_sum_of_heads(dev):
    q, k, v = qkv(1, 8, 128, 128, torch.float16, dev, hkv=2)
    q, k, v = (t.requires_grad_() for t in (q, k, v))
    out = cuda_llm.flash_attention(q, k, v, is_causal=True)
    out.float().sum().backward()
    torch.cuda.synchronize()
    qn, kn, vn = (to_np(t.detach()).astype(np.float64) for t in (q, k, v))
    on = to_np(out.detach()).astype(np.float64)
    lse = oracle.attention_lse(qn, kn, is_causal=True, dtype=np.float64)
    rq, rk, rv = oracle.attention_backward(np.ones_like(qn), qn, kn, vn, on, lse, is_causal=True,
                                           dtype=np.float64)
    for name, a, r in zip(("dq", "dk", "dv"), (q.grad, k.grad, v.grad), (rq, rk, rv)):
        _check_grad(a, r, name)


def test_backward_deterministic(dev):
    g = torch.Generator(device=dev).manual_seed(5)
    q, k, v = qkv(2, 4, 513, 128, torch.bfloat16, dev, gen=g)
    dout = torch.randn(2, 4, 513, 128, device=dev, generator=g).to(torch.bfloat16)
    out, lse = cuda_llm.flash_attention_forward_lse(q, k, v, is_causal=True)
    a = cuda_llm.flash_attention_backward(dout, q, k, v, out, lse, is_causal=True)
    b = cuda_llm.flash_attention_backward(dout, q, k, v, out, lse, is_causal=True)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_backward_single_key(dev):
    """S = 1: the softmax is constant, so dq = dk = 0 and dv = dout."""
    q, k, v = qkv(2, 4, 1, 128, torch.bfloat16, dev)
    dout = torch.randn_like(q)
    out, lse = cuda_llm.flash_attention_forward_lse(q, k, v)
    dq, dk, dv = cuda_llm.flash_attention_backward(dout, q, k, v, out, lse)
    torch.cuda.synchronize()
    assert dq.float().abs().max().item() < 1e-2 and dk.float().abs().max().item() < 1e-2
    assert torch.allclose(dv.float(), dout.float(), atol=1e-2, rtol=0)


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("b,hq,hkv,s", [(1, 2, 2, 64), (1, 2, 2, 100), (2, 4, 1, 300),
                                        (1, 2, 2, 1)])
@pytest.mark.parametrize("is_causal", [False, True])
def test_backward_float32(dev, head_dim, b, hq, hkv, s, is_causal):
    """The float32 instantiation (flash_attention_bwd_instantiations.cu:4):
    the reference grid plus GQA and S = 1, against the float64 oracle on the
    same inputs with the float32 forward's out and LSE, to 1e-3."""
    got, ref = _run_backward(b, hq, hkv, s, head_dim, torch.float32, dev, is_causal, seed=3)
    for name, a, r in zip(("dq", "dk", "dv"), got, ref):
        _check_grad(a, r, f"f32 {name}", atol=1e-3, rtol=1e-3, mean_abs=1e-4)


def test_autograd_float32(dev):
    q, k, v = qkv(1, 2, 200, 128, torch.float32, dev)
    q, k, v = (t.requires_grad_() for t in (q, k, v))
    out = cuda_llm.flash_attention(q, k, v, is_causal=True)
    dout = torch.randn_like(out)
    out.backward(dout)
    torch.cuda.synchronize()
    qn, kn, vn, dn = (to_np(t.detach()).astype(np.float64) for t in (q, k, v, dout))
    on = to_np(out.detach()).astype(np.float64)
    lse = oracle.attention_lse(qn, kn, is_causal=True, dtype=np.float64)
    ref = oracle.attention_backward(dn, qn, kn, vn, on, lse, is_causal=True, dtype=np.float64)
    for name, a, r in zip(("dq", "dk", "dv"), (q.grad, k.grad, v.grad), ref):
        _check_grad(a, r, f"f32 autograd {name}", atol=1e-3, rtol=1e-3, mean_abs=1e-4)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("b,h,s,is_causal", [(4, 16, 2304, True), (4, 16, 2048, True),
                                             (2, 8, 1100, False)])
def test_backward_large_paired_tiles(dev, b, h, s, is_causal, d):
    """Grids large enough for the causal launches to pair tiles per workgroup
    (9 tiles per head: the middle tiles of two heads make one work item); the
    kernel computes every head, sampled heads are checked against the oracle
    on the kernel forward's own out and LSE."""
    g = torch.Generator(device=dev).manual_seed(7)
    q, k, v = qkv(b, h, s, d, torch.bfloat16, dev, gen=g)
    dout = torch.randn(b, h, s, d, device=dev, generator=g).to(torch.bfloat16)
    out, lse = cuda_llm.flash_attention_forward_lse(q, k, v, is_causal=is_causal)
    dq, dk, dv = cuda_llm.flash_attention_backward(dout, q, k, v, out, lse, is_causal=is_causal)
    torch.cuda.synchronize()
    for bi, hi in [(0, 0), (b - 1, h - 1), (b // 2, h // 2 - 1)]:
        sel = lambda t: to_np(t[bi:bi + 1, hi:hi + 1]).astype(np.float64)
        ref = oracle.attention_backward(sel(dout), sel(q), sel(k), sel(v), sel(out),
                                        to_np(lse[bi:bi + 1, hi:hi + 1]).astype(np.float64),
                                        is_causal=is_causal, dtype=np.float64)
        for name, a, r in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
            _check_grad(a[bi:bi + 1, hi:hi + 1], r, f"{name} b{bi} h{hi}")


def test_backward_reference_benchmark_shape(dev):
    """The reference benchmark's backward shape (benchmark_pytorch.py:659-661:
    fp16, B = 2, H = 32, S = 4096, head dim 64, non-causal): every head is
    computed, two sampled heads are checked against the float64 oracle on the
    kernel forward's own out and LSE."""
    g = torch.Generator(device=dev).manual_seed(11)
    b, h, s, d = 2, 32, 4096, 64
    q, k, v = qkv(b, h, s, d, torch.float16, dev, gen=g)
    dout = torch.randn(b, h, s, d, device=dev, generator=g).to(torch.float16)
    out, lse = cuda_llm.flash_attention_forward_lse(q, k, v, is_causal=False)
    dq, dk, dv = cuda_llm.flash_attention_backward(dout, q, k, v, out, lse, is_causal=False)
    torch.cuda.synchronize()
    for bi, hi in [(0, 5), (1, 31)]:
        sel = lambda t: to_np(t[bi:bi + 1, hi:hi + 1]).astype(np.float64)
        ref = oracle.attention_backward(sel(dout), sel(q), sel(k), sel(v), sel(out),
                                        to_np(lse[bi:bi + 1, hi:hi + 1]).astype(np.float64),
                                        is_causal=False, dtype=np.float64)
        for name, a, r in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
            _check_grad(a[bi:bi + 1, hi:hi + 1], r, f"{name} b{bi} h{hi}")
