"""Paged KV-cache layout and paged decode — numpy restatement.

Test infrastructure only (see ``oracle/__init__.py``).

Reference anchors
-----------------
* layout   tests/_utils.py:105-133   cache[num_blocks, heads, head_dim, page] (page axis
           innermost); per-sequence logical block i lives at physical
           ``block_tables[n][i]``; physical blocks are a random permutation
* walk     paged_attention_kernel.cuh:61-76,86,127  token t of a sequence is in
           page ``block_tables[n][t // page]`` at ``cache[p][h][d][t % page]``;
           only ceil(L / page) table entries are read
* fp8      fp8_paged_attention_kernel.cuh:75-88  scale per head ``[H]`` or per
           (physical block, head) ``[num_blocks, H]``; k = code * k_scale,
           v = code * v_scale (the codes are e4m3 here, not int8 — the
           reference test's intended semantics, tests/test_kernels_misc.py:42-64)
* GQA      tests/_utils.py:67-72     kv head = q head // (Hq / Hkv)
* append   no reference kernel (the reference builds caches in torch, tests/
           _utils.py:105-133): token t of sequence n is written at the walk
           position above; FP8 pages are quantised with the per-page form of
           tests/test_kernels_misc.py:52-55
* L <= 0   writes zeros (the reference leaves the output unwritten,
           paged_attention_kernel.cuh:37-38; the l == 0 rule of
           flash_attention_v2_kernel.cuh:223 is applied instead)
"""
import numpy as np

from .attention import decode, default_scale
from .fp8 import e4m3_decode


def make_paged_cache(k, v, page_size, perm=None):
    """k, v: [N, Hkv, T, D] per-sequence contiguous caches.

    Returns (key_cache, value_cache [N*ceil(T/page), Hkv, D, page], block_tables
    int32 [N, ceil(T/page)]). ``perm`` (a permutation of the physical blocks)
    defaults to the identity.
    """
    k = np.asarray(k)
    v = np.asarray(v)
    n, h, t, d = k.shape
    bps = (t + page_size - 1) // page_size
    pad = bps * page_size - t
    if pad:
        k = np.pad(k, ((0, 0), (0, 0), (0, pad), (0, 0)))
        v = np.pad(v, ((0, 0), (0, 0), (0, pad), (0, 0)))
    kb = k.reshape(n, h, bps, page_size, d).transpose(0, 2, 1, 4, 3).reshape(n * bps, h, d, page_size)
    vb = v.reshape(n, h, bps, page_size, d).transpose(0, 2, 1, 4, 3).reshape(n * bps, h, d, page_size)
    num_blocks = n * bps
    perm = np.arange(num_blocks) if perm is None else np.asarray(perm)
    kc = np.empty_like(kb)
    vc = np.empty_like(vb)
    kc[perm] = kb
    vc[perm] = vb
    return kc, vc, perm.reshape(n, bps).astype(np.int32)


def gather_paged(cache, block_table_row, length, page_scale=None):
    """Walk one sequence's block table: -> [Hkv, length, D] (float32).

    ``page_scale``: optional per-page scale, [num_blocks, Hkv] or [Hkv]; when
    given, ``cache`` holds e4m3 codes that are decoded and multiplied by it.
    """
    cache = np.asarray(cache)
    page = cache.shape[-1]
    nb = (length + page - 1) // page
    ids = np.asarray(block_table_row[:nb], dtype=np.int64)
    pages = cache[ids]                                   # [nb, Hkv, D, page]
    if page_scale is not None:
        vals = e4m3_decode(pages)
        sc = np.asarray(page_scale, dtype=np.float32)
        if sc.ndim == 2:
            vals = vals * sc[ids][:, :, None, None]
        else:
            vals = vals * sc[None, :, None, None]
        pages = vals
    x = pages.astype(np.float32).transpose(1, 0, 3, 2)   # [Hkv, nb, page, D]
    x = x.reshape(x.shape[0], nb * page, x.shape[-1])
    return x[:, :length]


def paged_decode(query, key_cache, value_cache, block_tables, context_lens,
                 scale=None, k_scale=None, v_scale=None, dtype=np.float32):
    """Paged (optionally FP8) GQA decode -> [N, Hq, D] float.

    query [N, Hq, D]; caches [num_blocks, Hkv, D, page] (float, or uint8 e4m3
    codes when k_scale/v_scale are given); block_tables [N, max_blocks] int;
    context_lens [N] int.
    """
    query = np.asarray(query)
    n, hq, d = query.shape
    scale = default_scale(d) if scale is None else float(scale)
    hkv = np.asarray(key_cache).shape[1]
    out = np.zeros((n, hq, d), dtype=dtype)
    lens = np.asarray(context_lens).tolist()
    for i, L in enumerate(lens):
        L = int(L)
        if L <= 0:
            continue
        kk = gather_paged(key_cache, block_tables[i], L, k_scale)[None]
        vv = gather_paged(value_cache, block_tables[i], L, v_scale)[None]
        out[i] = decode(query[i][None], kk, vv, [L], scale=scale, dtype=dtype)[0]
    assert out.shape[1] % hkv == 0
    return out


def paged_append(key, value, key_cache, value_cache, block_tables, context_lens, new_lens=None,
                 k_scale=None, v_scale=None):
    """Append new tokens to a paged KV cache: the step before paged decode.

    key, value: [N, Hkv, T, D] new tokens; sequence n appends its first
    ``new_lens[n]`` (default T) tokens at positions context_lens[n] ..
    context_lens[n] + new_lens[n] - 1, token at position t going to
    ``cache[block_tables[n][t // 16]][h][:, t % 16]`` (the layout of
    tests/_utils.py:105-133). Positions past the block table and block ids
    outside the pool are skipped.

    * 16-bit caches (no scales): the new slots take the tokens as given.
    * FP8 caches (uint8 e4m3 codes) with per-head scales [Hkv]: the new slots
      take e4m3(x / s[h]), values beyond +-448 saturated.
    * FP8 caches with per-(page, head) scales [num_blocks, Hkv]: every page the
      append touches is quantised again over its valid slots (old slots
      decoded with the page's old scale, new slots as given), with scale =
      max(amax / 448, 1e-8) and codes e4m3(x / scale) — the recipe of
      tests/test_kernels_misc.py:52-55 applied per page, as the C4 benchmark
      cache is built; the page's unused slots are written as code 0.

    Returns new arrays (key_cache, value_cache, k_scale, v_scale); the scales
    are None for a 16-bit cache.
    """
    from .fp8 import E4M3_MAX, e4m3_encode

    key, value = np.asarray(key), np.asarray(value)
    kc, vc = np.array(key_cache, copy=True), np.array(value_cache, copy=True)
    fp8 = k_scale is not None
    ks = None if k_scale is None else np.array(k_scale, dtype=np.float32, copy=True)
    vs = None if v_scale is None else np.array(v_scale, dtype=np.float32, copy=True)
    n_seq, hkv, t_max, d = key.shape
    page = kc.shape[-1]
    max_blocks = block_tables.shape[1]
    num_blocks = kc.shape[0]
    lens = np.asarray(context_lens).astype(np.int64)
    news = np.full(n_seq, t_max) if new_lens is None else np.clip(np.asarray(new_lens), 0, t_max)

    def enc(x):
        x = np.clip(np.asarray(x, dtype=np.float32), -E4M3_MAX, E4M3_MAX)
        return e4m3_encode(x)

    for n in range(n_seq):
        lo = max(0, int(lens[n]))
        hi = min(lo + int(news[n]), max_blocks * page)
        if lo >= hi:
            continue
        for p in range(lo // page, (hi - 1) // page + 1):
            blk = int(block_tables[n, p])
            if blk < 0 or blk >= num_blocks:
                continue
            p0 = p * page
            for cache, src, sc in ((kc, key, ks), (vc, value, vs)):
                for h in range(hkv):
                    if not fp8:
                        for s in range(page):
                            pos = p0 + s
                            if lo <= pos < hi:
                                cache[blk, h, :, s] = src[n, h, pos - lo]
                    elif sc.ndim == 1:
                        for s in range(page):
                            pos = p0 + s
                            if lo <= pos < hi:
                                cache[blk, h, :, s] = enc(src[n, h, pos - lo].astype(np.float32)
                                                          / sc[h])
                    else:
                        vals = np.zeros((d, page), dtype=np.float32)
                        old_scale = sc[blk, h]
                        for s in range(page):
                            pos = p0 + s
                            if pos < lo:
                                vals[:, s] = e4m3_decode(cache[blk, h, :, s]) * old_scale
                            elif pos < hi:
                                vals[:, s] = src[n, h, pos - lo].astype(np.float32)
                        amax = np.abs(vals).max()
                        scale = np.float32(max(np.float32(amax) / np.float32(E4M3_MAX),
                                               np.float32(1e-8)))
                        codes = enc(vals / scale)
                        valid = (p0 + np.arange(page)) < hi
                        cache[blk, h] = np.where(valid[None, :], codes, 0).astype(np.uint8)
                        sc[blk, h] = scale
    return kc, vc, ks, vs
