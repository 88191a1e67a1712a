"""CPU tier: pin the oracle before trusting it.

Every oracle function is checked against something it does not share code
with: plain-Python float64 loops (golden fixtures and brute force), torch's
SDPA and float8 conversions, closed forms and invariants. A few checks plant a
mistake in the oracle (on the CPU) to show the check would catch it.
"""
import importlib
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from golden.make_golden import attend_rows

oattn = importlib.import_module("oracle.attention")

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def _case(g, name):
    pre = name + "/"
    return {k[len(pre):]: g[k] for k in g.files if k.startswith(pre)}


# ---------------------------------------------------------------------------
# golden vectors (float64 pure-Python loops)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("name", ["attn_causal_d64", "attn_full_d64", "attn_gqa_causal_d128"])
def test_attention_matches_golden(golden, name):
    c = _case(golden, name)
    out = oracle.attention(c["q"], c["k"], c["v"], is_causal=bool(c["causal"]))
    np.testing.assert_allclose(out, c["out"], atol=2e-6, rtol=0)


def test_paged_decode_matches_golden(golden):
    c = _case(golden, "paged_d64")
    out = oracle.paged_decode(c["query"], c["key_cache"], c["value_cache"], c["block_tables"],
                              c["context_lens"])
    np.testing.assert_allclose(out, c["out"], atol=2e-6, rtol=0)
    assert np.all(out[3] == 0)  # context length 0 -> zeros


def test_fp8_paged_decode_matches_golden(golden):
    c = _case(golden, "fp8_paged_d128")
    out = oracle.paged_decode(c["query"], c["key_cache"], c["value_cache"], c["block_tables"],
                              c["context_lens"], k_scale=c["k_scale"], v_scale=c["v_scale"])
    np.testing.assert_allclose(out, c["out"], atol=5e-6, rtol=0)


def test_mx_attention_matches_golden(golden):
    c = _case(golden, "mx_causal")
    deq = {n: oracle.mx_dequantize(c[n], c[n + "_scale"]) for n in "qkv"}
    out = oracle.attention(deq["q"], deq["k"], deq["v"], is_causal=bool(c["causal"]))
    np.testing.assert_allclose(out, c["out"], atol=1e-4 * max(1.0, np.abs(c["out"]).max()), rtol=0)


def test_planted_gqa_mistake_is_caught(golden, monkeypatch):
    """A wrong kv-head mapping (h % Hkv instead of h // group) must fail."""
    c = _case(golden, "attn_gqa_causal_d128")
    monkeypatch.setattr(oattn, "_kv_head", lambda h, hq, hkv: h % hkv)
    out = oracle.attention(c["q"], c["k"], c["v"], is_causal=True)
    assert np.abs(out - c["out"]).max() > 1e-2


def test_planted_causal_mistake_is_caught(golden):
    """Dropping the causal mask must fail the causal golden vector."""
    c = _case(golden, "attn_causal_d64")
    out = oracle.attention(c["q"], c["k"], c["v"], is_causal=False)
    assert np.abs(out - c["out"]).max() > 1e-2


# ---------------------------------------------------------------------------
# brute force and library cross-checks
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("s,d,causal", [(1, 8, True), (5, 8, False), (17, 16, True), (64, 8, False)])
def test_attention_vs_bruteforce(s, d, causal):
    rng = np.random.default_rng(s * 10 + d)
    q, k, v = (rng.standard_normal((1, 1, s, d)) for _ in range(3))
    ref = attend_rows(q[0, 0].tolist(), k[0, 0].tolist(), v[0, 0].tolist(), 1 / math.sqrt(d),
                      0 if causal else None)
    out = oracle.attention(q, k, v, is_causal=causal, dtype=np.float64)
    np.testing.assert_allclose(out[0, 0], np.array(ref), atol=1e-12, rtol=0)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("hq,hkv,s,d", [(4, 4, 100, 64), (8, 2, 77, 128), (4, 1, 256, 64)])
def test_attention_vs_torch_sdpa(causal, hq, hkv, s, d):
    g = torch.Generator().manual_seed(1)
    q = torch.randn(2, hq, s, d, generator=g)
    k = torch.randn(2, hkv, s, d, generator=g)
    v = torch.randn(2, hkv, s, d, generator=g)
    rep = hq // hkv
    ref = F.scaled_dot_product_attention(q, k.repeat_interleave(rep, 1), v.repeat_interleave(rep, 1),
                                         is_causal=causal)
    out = oracle.attention(q.numpy(), k.numpy(), v.numpy(), is_causal=causal)
    np.testing.assert_allclose(out, ref.numpy(), atol=2e-5, rtol=0)


def test_attention_c1_config():
    """BASELINE configs[0] (C1): fp32 q, k, v ~ N(0,1) [2, 8, 1024, 64], causal,
    scale 1/8 (tests/_utils.py:48-53 there). The fp32 oracle agrees with
    torch's CPU SDPA and with itself in float64 at that size, and its causal
    row 0 is v's row 0."""
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(2, 8, 1024, 64, generator=g) for _ in range(3))
    out = oracle.attention(q.numpy(), k.numpy(), v.numpy(), is_causal=True)
    assert out.dtype == np.float32 and out.shape == (2, 8, 1024, 64)
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    np.testing.assert_allclose(out, ref.numpy(), atol=2e-5, rtol=0)
    out64 = oracle.attention(q.numpy(), k.numpy(), v.numpy(), is_causal=True, dtype=np.float64)
    np.testing.assert_allclose(out, out64, atol=1e-5, rtol=0)
    np.testing.assert_array_equal(out[:, :, 0], v.numpy()[:, :, 0])


def test_lse_vs_torch():
    g = torch.Generator().manual_seed(2)
    q = torch.randn(1, 2, 50, 64, generator=g)
    k = torch.randn(1, 2, 50, 64, generator=g)
    s = (q @ k.transpose(-1, -2)) / 8.0
    s = s.masked_fill(~torch.ones(50, 50, dtype=torch.bool).tril(), float("-inf"))
    np.testing.assert_allclose(oracle.attention_lse(q.numpy(), k.numpy(), is_causal=True),
                               torch.logsumexp(s, -1).numpy(), atol=2e-5, rtol=0)


# ---------------------------------------------------------------------------
# invariants (closed forms)
# ---------------------------------------------------------------------------
def test_causal_first_row_is_first_value():
    rng = np.random.default_rng(3)
    q, k, v = (rng.standard_normal((2, 3, 40, 64)).astype(np.float32) for _ in range(3))
    out = oracle.attention(q, k, v, is_causal=True)
    np.testing.assert_allclose(out[:, :, 0], v[:, :, 0], atol=1e-6)


def test_constant_keys_give_prefix_mean():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((1, 1, 30, 64)).astype(np.float32)
    k = np.tile(rng.standard_normal((1, 1, 1, 64)).astype(np.float32), (1, 1, 30, 1))
    v = rng.standard_normal((1, 1, 30, 64)).astype(np.float32)
    out = oracle.attention(q, k, v, is_causal=True)
    means = np.cumsum(v[0, 0], axis=0) / np.arange(1, 31)[:, None]
    np.testing.assert_allclose(out[0, 0], means, atol=1e-5)


def test_zero_scale_gives_mean():
    rng = np.random.default_rng(5)
    q, k, v = (rng.standard_normal((1, 1, 20, 64)).astype(np.float32) for _ in range(3))
    out = oracle.attention(q, k, v, is_causal=False, scale=0.0)
    np.testing.assert_allclose(out[0, 0], np.broadcast_to(v[0, 0].mean(0), (20, 64)), atol=1e-5)


def test_key_permutation_invariance():
    rng = np.random.default_rng(6)
    q, k, v = (rng.standard_normal((1, 2, 33, 64)).astype(np.float32) for _ in range(3))
    p = rng.permutation(33)
    a = oracle.attention(q, k, v)
    b = oracle.attention(q, k[:, :, p], v[:, :, p])
    np.testing.assert_allclose(a, b, atol=1e-5)


# ---------------------------------------------------------------------------
# the kernels' blocking, restated on the CPU
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("s,qscale", [(100, 1.0), (300, 30.0), (129, 100.0)])
def test_tiled_online_softmax_equals_attention(causal, s, qscale):
    """Lazy rescaling (threshold 8 in log2 units) must be exact in fp32; large
    q scales force many rescale events."""
    rng = np.random.default_rng(s)
    q = (rng.standard_normal((1, 2, s, 64)) * qscale).astype(np.float32)
    k, v = (rng.standard_normal((1, 2, s, 64)).astype(np.float32) for _ in range(2))
    ref = oracle.attention(q, k, v, is_causal=causal, dtype=np.float64)
    out = oracle.attention_tiled(q, k, v, is_causal=causal)
    # fp32 logits of magnitude ~qscale*8 carry ~6e-8*|s| absolute rounding
    np.testing.assert_allclose(out, ref, atol=2e-5 * max(1.0, qscale / 5), rtol=0)


def test_split_merge_equals_full_attention():
    rng = np.random.default_rng(7)
    d, L = 64, 1000
    q = rng.standard_normal((1, 1, 1, d))
    k = rng.standard_normal((1, 1, L, d))
    v = rng.standard_normal((1, 1, L, d))
    full = oracle.attention(q, k, v, dtype=np.float64)[0, 0, 0]
    bounds = [0, 0, 100, 517, 1000, 1000]  # includes empty splits
    o_parts, l_parts = [], []
    for a, b in zip(bounds[:-1], bounds[1:]):
        o_parts.append(oracle.attention(q, k[:, :, a:b], v[:, :, a:b], dtype=np.float64)[0, 0, 0])
        l_parts.append(oracle.attention_lse(q, k[:, :, a:b], dtype=np.float64)[0, 0, 0] if b > a else -np.inf)
    merged = oracle.split_merge(np.array(o_parts), np.array(l_parts))
    np.testing.assert_allclose(merged, full, atol=1e-12)
    assert np.all(oracle.split_merge(np.zeros((2, d)), np.array([-np.inf, -np.inf])) == 0)


# ---------------------------------------------------------------------------
# paged layout
# ---------------------------------------------------------------------------
def test_paged_gather_roundtrip_is_bit_exact():
    rng = np.random.default_rng(8)
    n, h, t, d = 3, 2, 70, 64
    k = rng.standard_normal((n, h, t, d)).astype(np.float32)
    v = rng.standard_normal((n, h, t, d)).astype(np.float32)
    perm = rng.permutation(n * 5)
    kc, vc, bt = oracle.make_paged_cache(k, v, 16, perm=perm)
    assert kc.shape == (n * 5, h, d, 16)
    for i in range(n):
        assert np.array_equal(oracle.gather_paged(kc, bt[i], t), k[i])
        assert np.array_equal(oracle.gather_paged(vc, bt[i], t), v[i])


def test_paged_decode_equals_contiguous_decode():
    rng = np.random.default_rng(9)
    n, hq, hkv, t, d = 3, 8, 2, 50, 64
    q = rng.standard_normal((n, hq, d)).astype(np.float32)
    k = rng.standard_normal((n, hkv, t, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, t, d)).astype(np.float32)
    lens = np.array([50, 1, 33])
    kc, vc, bt = oracle.make_paged_cache(k, v, 16, perm=rng.permutation(n * 4))
    a = oracle.paged_decode(q, kc, vc, bt, lens)
    b = oracle.decode(q, k, v, lens)
    np.testing.assert_allclose(a, b, atol=1e-6)


# ---------------------------------------------------------------------------
# FP8 / MX codecs
# ---------------------------------------------------------------------------
def test_e4m3_decode_all_codes_vs_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    out = oracle.e4m3_decode(codes)
    assert np.array_equal(np.isnan(ref), np.isnan(out))
    assert np.array_equal(ref[~np.isnan(ref)], out[~np.isnan(out)])


def test_e4m3_encode_vs_torch():
    rng = np.random.default_rng(10)
    x = np.concatenate([
        np.linspace(-500, 500, 100001), rng.standard_normal(50000) * 50,
        rng.standard_normal(50000) * 1e-2, rng.standard_normal(20000) * 1e-3,
        # all representable values and every midpoint between neighbours (ties)
        oracle.e4m3_decode(np.arange(256, dtype=np.uint8)),
        [2.0 ** -10, 1.5 * 2.0 ** -9, 464.0, -464.0, 463.99, np.inf, -np.inf, np.nan, 0.0, -0.0],
    ]).astype(np.float32)
    vals = np.sort(np.unique(oracle.e4m3_decode(np.arange(256, dtype=np.uint8))))
    vals = vals[np.isfinite(vals)]
    x = np.concatenate([x, ((vals[1:] + vals[:-1]) / 2).astype(np.float32)])
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    out = oracle.e4m3_encode(x)
    assert np.array_equal(ref, out)


def test_e8m0_decode_vs_torch():
    b = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(b).view(torch.float8_e8m0fnu).float().numpy()
    out = oracle.e8m0_decode(b)
    assert np.array_equal(np.isnan(ref), np.isnan(out))
    assert np.array_equal(ref[~np.isnan(ref)], out[~np.isnan(out)])


def test_mx_quantize_closed_form():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((7, 128)) * rng.uniform(0.5, 4, (7, 128))).astype(np.float32)
    codes, sc = oracle.mx_quantize(x)
    amax = np.abs(x.reshape(7, 4, 32)).max(-1)
    assert np.array_equal(sc.astype(int) - 127, np.floor(np.log2(amax)).astype(int) - 8)
    deq = oracle.mx_dequantize(codes, sc)
    # elements within 2^-4 relative (e4m3 RNE) except saturated ones, which are <= 448 * X
    xs = x.reshape(7, 4, 32) / np.ldexp(1.0, sc.astype(int) - 127)[..., None]
    ok = np.abs(xs) <= 448
    rel = np.abs(deq.reshape(7, 4, 32) - x.reshape(7, 4, 32)) / np.maximum(np.abs(x.reshape(7, 4, 32)), 2.0 ** -6 * np.ldexp(1.0, sc.astype(int) - 127)[..., None])
    assert rel[ok].max() <= 2.0 ** -4 + 1e-7
    assert np.all(np.abs(deq.reshape(7, 4, 32)[~ok]) == 448 * np.ldexp(1.0, sc.astype(int) - 127)[..., None].repeat(32, -1)[~ok])


def test_mx_equal_scales_reduce_to_fp8():
    codes = np.arange(128, dtype=np.uint8).reshape(1, 128)
    codes[codes == 0x7F] = 0
    deq = oracle.mx_dequantize(codes, np.full((1, 4), 127, dtype=np.uint8))
    assert np.array_equal(deq, oracle.e4m3_decode(codes))


def test_per_page_quantization_matches_reference_recipe():
    g = torch.Generator().manual_seed(12)
    pages = torch.randn(5, 2, 64, 16, generator=g)
    codes, scale = oracle.quantize_per_page_fp8(pages.numpy())
    ref_scale = (pages.abs().amax(dim=(2, 3)) / 448.0).clamp_min(1e-8)
    ref_codes = (pages / ref_scale[:, :, None, None]).to(torch.float8_e4m3fn).view(torch.uint8)
    np.testing.assert_array_equal(scale, ref_scale.numpy())
    np.testing.assert_array_equal(codes, ref_codes.numpy())


# ---------------------------------------------------------------------------
# backward (flash_attention_bwd_kernel.cuh math)
# ---------------------------------------------------------------------------
def _torch_grads(q, k, v, dout, causal, scale=None):
    """fp64 torch autograd of SDPA with the GQA repeat: an implementation that
    shares no code with the oracle."""
    qt, kt, vt = (torch.from_numpy(x).double().requires_grad_() for x in (q, k, v))
    rep = q.shape[1] // k.shape[1]
    o = F.scaled_dot_product_attention(qt, kt.repeat_interleave(rep, 1), vt.repeat_interleave(rep, 1),
                                       is_causal=causal, scale=scale)
    o.backward(torch.from_numpy(dout).double())
    return o.detach().numpy(), qt.grad.numpy(), kt.grad.numpy(), vt.grad.numpy()


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("hq,hkv,s,d", [(2, 2, 64, 64), (2, 2, 100, 64), (4, 2, 37, 128), (3, 1, 5, 16)])
def test_backward_vs_torch_autograd(causal, hq, hkv, s, d):
    rng = np.random.default_rng(11)
    q = rng.standard_normal((1, hq, s, d))
    k = rng.standard_normal((1, hkv, s, d))
    v = rng.standard_normal((1, hkv, s, d))
    dout = rng.standard_normal((1, hq, s, d))
    o, gq, gk, gv = _torch_grads(q, k, v, dout, causal)
    lse = oracle.attention_lse(q, k, is_causal=causal, dtype=np.float64)
    dq, dk, dv = oracle.attention_backward(dout, q, k, v, o, lse, is_causal=causal, dtype=np.float64)
    for name, a, b in (("dq", dq, gq), ("dk", dk, gk), ("dv", dv, gv)):
        np.testing.assert_allclose(a, b, atol=1e-10, rtol=0, err_msg=name)


def test_backward_custom_scale_vs_torch_autograd():
    rng = np.random.default_rng(12)
    q, k, v, dout = (rng.standard_normal((1, 2, 33, 64)) for _ in range(4))
    o, gq, gk, gv = _torch_grads(q, k, v, dout, True, scale=0.3)
    lse = oracle.attention_lse(q, k, is_causal=True, scale=0.3, dtype=np.float64)
    dq, dk, dv = oracle.attention_backward(dout, q, k, v, o, lse, is_causal=True, scale=0.3,
                                           dtype=np.float64)
    for a, b in ((dq, gq), (dk, gk), (dv, gv)):
        np.testing.assert_allclose(a, b, atol=1e-10, rtol=0)


def test_backward_vs_finite_differences():
    """Central differences of the forward oracle, fp64, on a tiny case."""
    rng = np.random.default_rng(13)
    q, k, v, dout = (rng.standard_normal((1, 1, 4, 3)) for _ in range(4))
    for causal in (False, True):
        o = oracle.attention(q, k, v, is_causal=causal, dtype=np.float64)
        lse = oracle.attention_lse(q, k, is_causal=causal, dtype=np.float64)
        grads = oracle.attention_backward(dout, q, k, v, o, lse, is_causal=causal, dtype=np.float64)
        eps = 1e-6
        for which, g in zip(range(3), grads):
            x = [q, k, v][which]
            num = np.zeros_like(x)
            for idx in np.ndindex(x.shape):
                xp, xm = x.copy(), x.copy()
                xp[idx] += eps
                xm[idx] -= eps
                args_p = [q, k, v]
                args_m = [q, k, v]
                args_p[which], args_m[which] = xp, xm
                fp = (oracle.attention(*args_p, is_causal=causal, dtype=np.float64) * dout).sum()
                fm = (oracle.attention(*args_m, is_causal=causal, dtype=np.float64) * dout).sum()
                num[idx] = (fp - fm) / (2 * eps)
            np.testing.assert_allclose(g, num, atol=1e-7, rtol=0)


def test_backward_single_key_closed_form():
    """One key: the softmax is constant 1, so dq = dk = 0 and dv = dout."""
    rng = np.random.default_rng(14)
    q, k, v, dout = (rng.standard_normal((2, 2, 1, 64)) for _ in range(4))
    o = oracle.attention(q, k, v, dtype=np.float64)
    lse = oracle.attention_lse(q, k, dtype=np.float64)
    dq, dk, dv = oracle.attention_backward(dout, q, k, v, o, lse, dtype=np.float64)
    assert np.abs(dq).max() < 1e-12 and np.abs(dk).max() < 1e-12
    np.testing.assert_allclose(dv, dout, atol=1e-12, rtol=0)


def test_planted_backward_mistake_is_caught(monkeypatch):
    """Dropping the D_i term (a plausible slip) breaks the autograd check."""
    rng = np.random.default_rng(15)
    q, k, v, dout = (rng.standard_normal((1, 2, 20, 16)) for _ in range(4))
    o, gq, _, _ = _torch_grads(q, k, v, dout, True)
    lse = oracle.attention_lse(q, k, is_causal=True, dtype=np.float64)
    real = oattn.attention_backward

    def dropped_d(dout_, q_, k_, v_, out_, lse_, **kw):
        return real(dout_, q_, k_, v_, np.zeros_like(out_), lse_, **kw)

    monkeypatch.setattr(oattn, "attention_backward", dropped_d)
    dq, _, _ = oattn.attention_backward(dout, q, k, v, o, lse, is_causal=True, dtype=np.float64)
    assert np.abs(dq - gq).max() > 1e-3


# ---------------------------------------------------------------------------
# paged append
# ---------------------------------------------------------------------------
def _append_case(rng, n=3, hkv=2, d=16, lens=(37, 16, 5), extra=4):
    t = max(lens)
    k = rng.standard_normal((n, hkv, t, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, t, d)).astype(np.float32)
    bps = (t + 15) // 16 + extra
    perm = rng.permutation(n * bps)
    tables = perm.reshape(n, bps).astype(np.int32)
    return k, v, tables, np.asarray(lens)


def test_append_whole_sequences_equals_make_paged_cache():
    rng = np.random.default_rng(21)
    k, v, tables, lens = _append_case(rng, extra=0)
    n, hkv, t, d = k.shape
    kc0 = np.zeros((tables.size, hkv, d, 16), np.float32)
    kc, vc, _, _ = oracle.paged_append(k, v, kc0, kc0, tables, np.zeros(n, np.int32), lens)
    ref_k, ref_v, _ = oracle.make_paged_cache(k, v, 16, perm=tables.reshape(-1))
    for i in range(n):
        for p in range((lens[i] + 15) // 16):
            blk = tables[i, p]
            for s in range(16):
                if p * 16 + s < lens[i]:
                    np.testing.assert_array_equal(kc[blk, :, :, s], ref_k[blk, :, :, s])
                    np.testing.assert_array_equal(vc[blk, :, :, s], ref_v[blk, :, :, s])


def test_append_token_by_token_equals_all_at_once():
    rng = np.random.default_rng(22)
    k, v, tables, lens = _append_case(rng)
    n, hkv, t, d = k.shape
    zero = np.zeros((tables.size, hkv, d, 16), np.float32)
    full_k, full_v, _, _ = oracle.paged_append(k, v, zero, zero, tables, np.zeros(n, np.int32), lens)
    kc, vc = zero.copy(), zero.copy()
    for step in range(t):
        new = (lens > step).astype(np.int32)
        kc, vc, _, _ = oracle.paged_append(k[:, :, step:step + 1], v[:, :, step:step + 1], kc, vc,
                                           tables, np.minimum(lens, step), new)
    np.testing.assert_array_equal(kc, full_k)
    np.testing.assert_array_equal(vc, full_v)


def test_append_fp8_per_page_equals_reference_recipe():
    """Whole sequences into empty pages == quantize_per_page_fp8 of the paged
    cache (the reference recipe, per page), unused slots zero."""
    rng = np.random.default_rng(23)
    k, v, tables, lens = _append_case(rng, extra=0)
    n, hkv, t, d = k.shape
    kz = np.zeros((tables.size, hkv, d, 16), np.uint8)
    sz = np.ones((tables.size, hkv), np.float32)
    kc, vc, ks, vs = oracle.paged_append(k, v, kz, kz, tables, np.zeros(n, np.int32), lens,
                                         k_scale=sz, v_scale=sz)
    masked_k = k.copy()
    masked_v = v.copy()
    for i in range(n):
        masked_k[i, :, lens[i]:] = 0
        masked_v[i, :, lens[i]:] = 0
    pk, pv, _ = oracle.make_paged_cache(masked_k, masked_v, 16, perm=tables.reshape(-1))
    ck, sk = oracle.quantize_per_page_fp8(pk)
    cv, sv = oracle.quantize_per_page_fp8(pv)
    np.testing.assert_array_equal(kc, ck)
    np.testing.assert_array_equal(vc, cv)
    used = np.concatenate([tables[i, :(lens[i] + 15) // 16] for i in range(n)])
    np.testing.assert_array_equal(ks[used], sk[used])  # pages never touched keep their scale
    np.testing.assert_array_equal(vs[used], sv[used])


def test_append_fp8_per_page_incremental_when_first_chunk_holds_the_max():
    """If a page's first append already holds its largest magnitude, appending
    the rest later re-derives the same codes: equal to one append, bit-exact."""
    rng = np.random.default_rng(24)
    k, v, tables, lens = _append_case(rng, lens=(32, 32, 32), extra=0)
    k[:, :, 0::16, 0] = 50.0  # slot 0 of every page carries the page max
    v[:, :, 0::16, 0] = -50.0
    n, hkv, t, d = k.shape
    kz = np.zeros((tables.size, hkv, d, 16), np.uint8)
    sz = np.ones((tables.size, hkv), np.float32)
    one = oracle.paged_append(k, v, kz, kz, tables, np.zeros(n, np.int32), lens, k_scale=sz, v_scale=sz)
    a = oracle.paged_append(k[:, :, :5], v[:, :, :5], kz, kz, tables, np.zeros(n, np.int32), None,
                            k_scale=sz, v_scale=sz)
    b = oracle.paged_append(k[:, :, 5:], v[:, :, 5:], a[0], a[1], tables, np.full(n, 5, np.int32),
                            None, k_scale=a[2], v_scale=a[3])
    for x, y in zip(one, b):
        np.testing.assert_array_equal(x, y)


def test_append_fp8_per_head_equals_reference_recipe():
    rng = np.random.default_rng(25)
    k, v, tables, lens = _append_case(rng, extra=0)
    n, hkv, t, d = k.shape
    s = np.array([0.01, 0.02], np.float32)
    kz = np.zeros((tables.size, hkv, d, 16), np.uint8)
    kc, _, _, _ = oracle.paged_append(k, v, kz, kz, tables, np.zeros(n, np.int32), lens,
                                      k_scale=s, v_scale=s)
    for i in range(n):
        for pos in range(lens[i]):
            blk, slot = tables[i, pos // 16], pos % 16
            for h in range(hkv):
                want = torch.from_numpy(np.clip(k[i, h, pos] / s[h], -448, 448)).to(
                    torch.float8_e4m3fn).view(torch.uint8).numpy()
                np.testing.assert_array_equal(kc[blk, h, :, slot], want)


def test_append_skips_out_of_range_blocks_and_positions():
    rng = np.random.default_rng(26)
    k, v, tables, _ = _append_case(rng, lens=(20, 20, 20), extra=0)
    n, hkv, t, d = k.shape
    tables = tables.copy()
    tables[0, 1] = -1          # invalid block: its tokens are dropped
    zero = np.zeros((tables.size, hkv, d, 16), np.float32)
    kc, _, _, _ = oracle.paged_append(k, v, zero, zero, tables, np.array([0, 20, 30]), None)
    # sequence 0: page 1 (positions 16..31) has block -1 and is dropped
    np.testing.assert_array_equal(kc[tables[0, 0], :, :, :], k[0, :, :16].transpose(0, 2, 1))
    # sequence 1 (table of 2 pages = 32 positions): positions 20..31 fit, 32..39 are dropped
    # sequence 2 starts at 30: positions 30, 31 fit
    blk = tables[1, 1]
    np.testing.assert_array_equal(kc[blk, :, :, 4:16], k[1, :, :12].transpose(0, 2, 1))
    assert np.all(kc[tables[1, 0]] == 0)
    np.testing.assert_array_equal(kc[tables[2, 1], :, :, 14:16], k[2, :, :2].transpose(0, 2, 1))


# ---------------------------------------------------------------------------
# RoPE (rotate-half, tests/_utils.py:75-94)
# ---------------------------------------------------------------------------
def _rope_tables(s, d, base=10000.0):
    """cos / sin [S, D] as tests/_utils.py:75-81 builds them."""
    inv = 1.0 / (base ** (np.arange(0, d, 2, dtype=np.float64) / d))
    ang = np.outer(np.arange(s, dtype=np.float64), inv)
    emb = np.concatenate([ang, ang], axis=-1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32), ang


def test_rope_equals_complex_rotation():
    """Rotate-half RoPE is the complex product (x_c + i x_{c+D/2}) e^{i theta_c}."""
    rng = np.random.default_rng(31)
    s, d = 50, 64
    x = rng.standard_normal((2, 3, s, d)).astype(np.float32)
    cos, sin, ang = _rope_tables(s, d)
    got = oracle.apply_rope(x, cos, sin)
    z = (x[..., : d // 2] + 1j * x[..., d // 2:]) * np.exp(1j * ang)
    want = np.concatenate([z.real, z.imag], axis=-1)
    np.testing.assert_allclose(got, want, atol=2e-5, rtol=0)


def test_rope_preserves_pair_norms_and_position_zero():
    rng = np.random.default_rng(32)
    s, d = 40, 128
    x = rng.standard_normal((1, 2, s, d)).astype(np.float32)
    cos, sin, _ = _rope_tables(s, d)
    y = oracle.apply_rope(x, cos, sin)
    h = d // 2
    np.testing.assert_allclose(x[..., :h] ** 2 + x[..., h:] ** 2, y[..., :h] ** 2 + y[..., h:] ** 2,
                               rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(y[:, :, 0], x[:, :, 0], atol=0, rtol=0)


@pytest.mark.parametrize("causal", [False, True])
def test_rope_attention_vs_torch_sdpa(causal):
    rng = np.random.default_rng(33)
    s, d = 70, 64
    q, k, v = (rng.standard_normal((1, 4, s, d)).astype(np.float32) for _ in range(3))
    cos, sin, _ = _rope_tables(s, d)
    tq, tk = (torch.from_numpy(x) for x in (q, k))
    tc, ts = torch.from_numpy(cos), torch.from_numpy(sin)
    rot = lambda t: torch.cat([-t[..., d // 2:], t[..., : d // 2]], dim=-1)  # noqa: E731
    ref = F.scaled_dot_product_attention(tq * tc + rot(tq) * ts, tk * tc + rot(tk) * ts,
                                         torch.from_numpy(v), is_causal=causal)
    np.testing.assert_allclose(oracle.rope_attention(q, k, v, cos, sin, is_causal=causal),
                               ref.numpy(), atol=2e-5, rtol=0)
