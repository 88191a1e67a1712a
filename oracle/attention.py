"""fp32 attention math — restatement of the reference's torch oracles in numpy.

Test infrastructure only (see ``oracle/__init__.py``).

Reference anchors
-----------------
* ``ref_attention``  tests/_utils.py:48-53   softmax(q k^T * scale [+ causal]) v in fp32
* causal mask        tests/_utils.py:60-63   ``ones(sq, sk).tril()`` (top-left aligned)
* GQA mapping        tests/_utils.py:67-72   ``repeat_interleave(group)`` => kv head = h // group
* ``ref_decode``     tests/_utils.py:136-142 per-sequence prefix of ``context_lens[n]`` keys
* default scale      fused_softmax_binding.cpp:69-72  1/sqrt(head_dim)
* empty softmax row  flash_attention_v2_kernel.cuh:223  l == 0 -> output 0
* online softmax     flash_attention_v2_kernel.cuh:179-229 (running max / sum)
* RoPE               tests/_utils.py:75-94 (rotate-half tables and rotation)
* backward           flash_attention_bwd_kernel.cuh:9-19, 96-214 (dQ, dK, dV from
                     the forward's LSE; D_i = rowsum(dO * O))
"""
import math

import numpy as np

LOG2E = 1.4426950408889634


def default_scale(head_dim):
    """1/sqrt(D), the binding's default (fused_softmax_binding.cpp:69-72)."""
    return 1.0 / math.sqrt(head_dim)


def _kv_head(h, hq, hkv):
    if hq % hkv:
        raise ValueError(f"num q heads {hq} not a multiple of num kv heads {hkv}")
    return h // (hq // hkv)


def _row_attention(qh, kh, vh, is_causal, scale, dtype, q_block, q_offset=0,
                   want_lse=False):
    """One (b, h) slice: qh [Sq, D], kh/vh [Skv, D] -> ([Sq, D], lse [Sq])."""
    sq, d = qh.shape
    skv = kh.shape[0]
    out = np.zeros((sq, vh.shape[1]), dtype=dtype)
    lse = np.full((sq,), -np.inf, dtype=dtype)
    if skv == 0 or sq == 0:
        return out, lse
    kt = np.ascontiguousarray(kh.T.astype(dtype, copy=False))
    vv = vh.astype(dtype, copy=False)
    for r0 in range(0, sq, q_block):
        r1 = min(sq, r0 + q_block)
        qb = qh[r0:r1].astype(dtype, copy=False)
        # causal: key j visible to query i iff j <= i (+ q_offset); top-left tril
        kend = skv if not is_causal else min(skv, r1 + q_offset)
        if kend <= 0:
            continue
        s = (qb @ kt[:, :kend]) * dtype(scale)
        if is_causal:
            rows = np.arange(r0, r1)[:, None] + q_offset
            cols = np.arange(kend)[None, :]
            s = np.where(cols <= rows, s, -np.inf)
        m = s.max(axis=1, keepdims=True)
        valid = np.isfinite(m)
        m_safe = np.where(valid, m, 0).astype(dtype)
        p = np.exp(s - m_safe)
        l = p.sum(axis=1, keepdims=True)
        o = p @ vv[:kend]
        inv = np.where(l > 0, 1.0 / np.where(l > 0, l, 1), 0).astype(dtype)
        out[r0:r1] = o * inv
        if want_lse:
            with np.errstate(divide="ignore"):
                lse[r0:r1] = np.where(l[:, 0] > 0, m_safe[:, 0] + np.log(l[:, 0]), -np.inf)
    return out, lse


def attention(q, k, v, is_causal=False, scale=None, dtype=np.float32,
              q_block=512, heads=None):
    """softmax(q k^T * scale + mask) v.

    q: [B, Hq, Sq, D]; k, v: [B, Hkv, Skv, D] with Hq % Hkv == 0.
    Returns [B, Hq, Sq, Dv] in ``dtype`` (float32 by default, as the
    reference's oracle; float64 for pinning).
    ``heads``: optional list of (b, h) pairs to compute (others stay zero);
    used by the CPU baseline to time a bounded sample.
    """
    q = np.asarray(q)
    k = np.asarray(k)
    v = np.asarray(v)
    b, hq, sq, d = q.shape
    hkv = k.shape[1]
    scale = default_scale(d) if scale is None else float(scale)
    out = np.zeros((b, hq, sq, v.shape[-1]), dtype=dtype)
    pairs = heads if heads is not None else [(i, h) for i in range(b) for h in range(hq)]
    for (i, h) in pairs:
        kh = _kv_head(h, hq, hkv)
        out[i, h], _ = _row_attention(q[i, h], k[i, kh], v[i, kh], is_causal,
                                      scale, dtype, q_block)
    return out


def attention_lse(q, k, is_causal=False, scale=None, dtype=np.float32):
    """Natural-log logsumexp of the scaled, masked scores [B, Hq, Sq]
    (tests/_utils.py:56-64, ``ref_lse``)."""
    q = np.asarray(q)
    k = np.asarray(k)
    b, hq, sq, d = q.shape
    hkv = k.shape[1]
    scale = default_scale(d) if scale is None else float(scale)
    lse = np.zeros((b, hq, sq), dtype=dtype)
    for i in range(b):
        for h in range(hq):
            kh = _kv_head(h, hq, hkv)
            _, lse[i, h] = _row_attention(q[i, h], k[i, kh], k[i, kh], is_causal,
                                          scale, dtype, 512, want_lse=True)
    return lse


def attention_backward(dout, q, k, v, out, lse, is_causal=False, scale=None,
                       dtype=np.float32):
    """Gradients (dq, dk, dv) of O = softmax(q k^T * scale + mask) v, given the
    forward output ``out`` and its natural-log row logsumexp ``lse``.

    Restates the reference backward (flash_attention_bwd_kernel.cuh): D_i =
    rowsum(dO * O) (:96-108); P = exp(S * scale - LSE_i) (:166-172); dP = dO
    V^T (:174-181); dS = P (dP - D_i) * scale (:183-184); dQ = dS K
    (:188-199); dV = P^T dO and dK = dS^T Q (:201-214). Masked entries (key >
    query when causal) have P = dS = 0 (:160-163). GQA (Hkv < Hq, kv head =
    h // (Hq / Hkv)): dk and dv of a kv head are the sums over its q heads,
    the gradient of the repeat_interleave in tests/_utils.py:67-72.

    dout, q, out: [B, Hq, S, D]; k, v: [B, Hkv, S, D]; lse: [B, Hq, S].
    """
    dout, q, k, v, out, lse = (np.asarray(x) for x in (dout, q, k, v, out, lse))
    b, hq, sq, d = q.shape
    hkv, skv = k.shape[1], k.shape[2]
    scale = default_scale(d) if scale is None else float(scale)
    dq = np.zeros(q.shape, dtype=dtype)
    dk = np.zeros(k.shape, dtype=dtype)
    dv = np.zeros(v.shape, dtype=dtype)
    for i in range(b):
        for h in range(hq):
            kh = _kv_head(h, hq, hkv)
            qh, kk, vv = (x.astype(dtype) for x in (q[i, h], k[i, kh], v[i, kh]))
            do, oh = dout[i, h].astype(dtype), out[i, h].astype(dtype)
            s = (qh @ kk.T) * dtype(scale)
            visible = np.ones((sq, skv), dtype=bool)
            if is_causal:
                visible = np.arange(skv)[None, :] <= np.arange(sq)[:, None]
            with np.errstate(invalid="ignore", over="ignore"):
                p = np.where(visible, np.exp(s - lse[i, h].astype(dtype)[:, None]), 0)
            p = np.nan_to_num(p, nan=0.0).astype(dtype)
            d_row = (do * oh).sum(axis=1, keepdims=True)
            dp = do @ vv.T
            ds = (p * (dp - d_row) * dtype(scale)).astype(dtype)
            dq[i, h] = ds @ kk
            dk[i, kh] += ds.T @ qh
            dv[i, kh] += p.T @ do
    return dq, dk, dv


def apply_rope(x, cos, sin):
    """Rotate-half RoPE (tests/_utils.py:84-89, ``apply_rope``; kernel
    fused_rope_flash_attention_kernel.cuh:60-70,98-108): x [..., S, D],
    cos / sin [S, D] -> x * cos + rot(x) * sin with rot(x) = [-x[D/2:], x[:D/2]],
    in float32."""
    x = np.asarray(x, dtype=np.float32)
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return (x * np.asarray(cos, dtype=np.float32) + rot * np.asarray(sin, dtype=np.float32)).astype(
        np.float32)


def rope_attention(q, k, v, cos, sin, is_causal=True, scale=None, dtype=np.float32):
    """Attention on RoPE-rotated q and k (tests/_utils.py:92-94,
    ``ref_rope_attention``)."""
    return attention(apply_rope(q, cos, sin), apply_rope(k, cos, sin), v, is_causal=is_causal,
                     scale=scale, dtype=dtype)


def decode(q, k, v, context_lens, scale=None, dtype=np.float32):
    """q_len = 1 attention over the first ``context_lens[n]`` keys.

    q: [N, Hq, D]; k, v: [N, Hkv, T, D]; context_lens: [N] ints.
    Restates ``ref_decode`` (tests/_utils.py:136-142) with the GQA mapping of
    tests/_utils.py:67-72. A sequence with L <= 0 yields zeros (the l == 0 rule,
    flash_attention_v2_kernel.cuh:223).
    """
    q = np.asarray(q)
    n, hq, d = q.shape
    hkv = k.shape[1]
    scale = default_scale(d) if scale is None else float(scale)
    out = np.zeros((n, hq, v.shape[-1]), dtype=dtype)
    for i, L in enumerate(np.asarray(context_lens).tolist()):
        L = max(0, int(L))
        for h in range(hq):
            kh = _kv_head(h, hq, hkv)
            o, _ = _row_attention(q[i, h][None], k[i, kh, :L], v[i, kh, :L],
                                  False, scale, dtype, 1)
            out[i, h] = o[0]
    return out


def attention_tiled(q, k, v, is_causal=False, scale=None, block_m=128,
                    block_n=64, rescale_threshold=8.0, p_round=None):
    """Restatement of the HIP prefill kernel's blocking (fp32).

    Per query tile of ``block_m`` rows the kernel walks key tiles of
    ``block_n`` up to the causal diagonal (flash_attention_v2_kernel.cuh:82-83),
    keeps a running max ``m`` and sum ``l`` per row in the log2 domain
    (scores pre-multiplied by scale*log2(e)), and only rescales the output
    accumulator when a row's tile max exceeds ``m`` by more than
    ``rescale_threshold`` (in log2 units) — between rescales p = 2^(s - m) may
    grow up to 2^threshold, which fp32 absorbs exactly in the final o / l.
    ``p_round`` optionally models the bf16 rounding of P before the PV product.
    """
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    b, hq, s_q, d = q.shape
    hkv, s_kv = k.shape[1], k.shape[2]
    scale = default_scale(d) if scale is None else float(scale)
    c = np.float32(scale * LOG2E)
    out = np.zeros((b, hq, s_q, v.shape[-1]), dtype=np.float32)
    for i in range(b):
        for h in range(hq):
            kh = _kv_head(h, hq, hkv)
            for r0 in range(0, s_q, block_m):
                r1 = min(s_q, r0 + block_m)
                qb = q[i, h, r0:r1]
                m = np.full((r1 - r0,), -np.inf, dtype=np.float32)
                l = np.zeros((r1 - r0,), dtype=np.float32)
                acc = np.zeros((r1 - r0, v.shape[-1]), dtype=np.float32)
                kend = s_kv if not is_causal else min(s_kv, r1)
                for c0 in range(0, kend, block_n):
                    c1 = min(kend, c0 + block_n)
                    sblk = (qb @ k[i, kh, c0:c1].T) * c
                    if is_causal:
                        rows = np.arange(r0, r1)[:, None]
                        cols = np.arange(c0, c1)[None, :]
                        sblk = np.where(cols <= rows, sblk, -np.inf)
                    tmax = sblk.max(axis=1)
                    need = tmax > m + rescale_threshold
                    if need.any():
                        m_new = np.maximum(m, tmax)
                        alpha = np.where(np.isfinite(m), np.exp2(m - np.where(np.isfinite(m_new), m_new, 0)), 0).astype(np.float32)
                        alpha = np.where(np.isfinite(m_new), alpha, 1).astype(np.float32)
                        acc *= alpha[:, None]
                        l *= alpha
                        m = m_new
                    m_safe = np.where(np.isfinite(m), m, 0).astype(np.float32)
                    p = np.exp2(sblk - m_safe[:, None]).astype(np.float32)
                    l += p.sum(axis=1)
                    pp = p if p_round is None else p_round(p)
                    acc += pp @ v[i, kh, c0:c1]
                inv = np.where(l > 0, 1.0 / np.where(l > 0, l, 1), 0).astype(np.float32)
                out[i, h, r0:r1] = acc * inv[:, None]
    return out


def split_merge(o_parts, lse_parts):
    """Log-sum-exp merge of split-K partial results.

    o_parts: [..., n_split, D] normalised partial outputs; lse_parts:
    [..., n_split] natural-log partial logsumexps (-inf for an empty split).
    Returns [..., D]: sum_i exp(lse_i - LSE) o_i with LSE = logsumexp_i lse_i,
    or 0 when every split is empty (the l == 0 rule).
    The reference walks a whole context in one block
    (paged_attention_kernel.cuh:68); splitting it is this build's single-GPU
    form of context parallelism, and this function is its specification.
    """
    o_parts = np.asarray(o_parts, dtype=np.float64)
    lse_parts = np.asarray(lse_parts, dtype=np.float64)
    mx = lse_parts.max(axis=-1, keepdims=True)
    finite = np.isfinite(mx)
    mx_safe = np.where(finite, mx, 0)
    w = np.where(np.isfinite(lse_parts), np.exp(lse_parts - mx_safe), 0)
    tot = w.sum(axis=-1, keepdims=True)
    w = np.where(tot > 0, w / np.where(tot > 0, tot, 1), 0)
    return (w[..., None] * o_parts).sum(axis=-2)
