"""Generate the committed golden vectors in ``tests/golden/golden.npz``.

The expected outputs are computed by plain-Python float64 loops written
independently of ``oracle/`` (no numpy linear algebra), on tiny inputs whose
values are exactly representable in bf16 (and, for the FP8 / MX cases, given as
e4m3 codes + scales), so the same vectors pin the CPU oracle and the gfx950
kernels. The reference ships no golden vectors of its own (its tests compare
against torch SDPA on random inputs, tests/_utils.py:48-53), so these are
derived from the specification those tests state:

* attention: softmax(q k^T * scale [+ causal tril]) v, scale = 1/sqrt(D)
  (tests/_utils.py:48-64, fused_softmax_binding.cpp:69-72), GQA kv head =
  h // (Hq/Hkv) (tests/_utils.py:67-72);
* paged decode: tokens gathered through block tables from
  cache[block][head][d][t % 16] (tests/_utils.py:105-142);
* fp8 paged decode: k = e4m3(code) * scale[block, head]
  (tests/test_kernels_misc.py:42-64, fused_softmax_binding.cpp:640,671);
* MXFP8: x = e4m3(code) * 2^(e8m0 - 127) per 32 elements of D (OCP MX v1.0).

Run: ``python tests/golden/make_golden.py`` (deterministic; seed 0).
"""
import math
import os
import struct

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")


def bf16_round(x):
    """Round float32 values to the nearest bf16 (ties to even), kept as float32."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def e4m3_value(code):
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 7
    if e == 15 and m == 7:
        return float("nan")
    if e == 0:
        return s * m * 2.0 ** -9
    return s * (1 + m / 8.0) * 2.0 ** (e - 7)


def attend_rows(q_rows, k_rows, v_rows, scale, causal_offset=None):
    """Pure-Python float64 softmax attention for a list of query rows."""
    out = []
    for i, q in enumerate(q_rows):
        n_keys = len(k_rows) if causal_offset is None else min(len(k_rows), i + causal_offset + 1)
        logits = [sum(a * b for a, b in zip(q, k_rows[j])) * scale for j in range(n_keys)]
        if not logits:
            out.append([0.0] * len(v_rows[0]) if v_rows else [])
            continue
        m = max(logits)
        w = [math.exp(x - m) for x in logits]
        tot = sum(w)
        out.append([sum(w[j] * v_rows[j][d] for j in range(n_keys)) / tot
                    for d in range(len(v_rows[0]))])
    return out


def case_attention(rng, b, hq, hkv, s, d, causal):
    q = bf16_round(rng.standard_normal((b, hq, s, d)).astype(np.float32))
    k = bf16_round(rng.standard_normal((b, hkv, s, d)).astype(np.float32))
    v = bf16_round(rng.standard_normal((b, hkv, s, d)).astype(np.float32))
    scale = 1.0 / math.sqrt(d)
    out = np.zeros((b, hq, s, d))
    for i in range(b):
        for h in range(hq):
            kh = h // (hq // hkv)
            out[i, h] = attend_rows(q[i, h].tolist(), k[i, kh].tolist(), v[i, kh].tolist(),
                                    scale, 0 if causal else None)
    return dict(q=q, k=k, v=v, out=out, causal=np.array(causal))


def case_paged(rng, lens, hq, hkv, d, fp8):
    page = 16
    n = len(lens)
    pages_per_seq = [(L + page - 1) // page for L in lens]
    n_blocks = sum(pages_per_seq) + 3          # a few unused blocks
    perm = rng.permutation(n_blocks)
    max_blocks = max(pages_per_seq + [1])
    tables = np.zeros((n, max_blocks), dtype=np.int32)
    cursor = 0
    for i, nb in enumerate(pages_per_seq):
        tables[i, :nb] = perm[cursor:cursor + nb]
        cursor += nb
    q = bf16_round(rng.standard_normal((n, hq, d)).astype(np.float32))
    if fp8:
        # codes drawn from finite e4m3 values (no NaN), scales per (block, head)
        finite = [c for c in range(256) if (c & 0x7F) != 0x7F]
        kc = rng.choice(finite, size=(n_blocks, hkv, d, page)).astype(np.uint8)
        vc = rng.choice(finite, size=(n_blocks, hkv, d, page)).astype(np.uint8)
        ks = (rng.uniform(0.5, 2.0, size=(n_blocks, hkv)) / 448.0).astype(np.float32)
        vs = (rng.uniform(0.5, 2.0, size=(n_blocks, hkv)) / 448.0).astype(np.float32)
        kval = lambda blk, h, dd, t: e4m3_value(int(kc[blk, h, dd, t])) * float(ks[blk, h])
        vval = lambda blk, h, dd, t: e4m3_value(int(vc[blk, h, dd, t])) * float(vs[blk, h])
    else:
        kc = bf16_round(rng.standard_normal((n_blocks, hkv, d, page)).astype(np.float32))
        vc = bf16_round(rng.standard_normal((n_blocks, hkv, d, page)).astype(np.float32))
        kval = lambda blk, h, dd, t: float(kc[blk, h, dd, t])
        vval = lambda blk, h, dd, t: float(vc[blk, h, dd, t])
    scale = 1.0 / math.sqrt(d)
    out = np.zeros((n, hq, d))
    for i, L in enumerate(lens):
        for h in range(hq):
            kh = h // (hq // hkv)
            krows, vrows = [], []
            for t in range(L):
                blk = int(tables[i, t // page])
                krows.append([kval(blk, kh, dd, t % page) for dd in range(d)])
                vrows.append([vval(blk, kh, dd, t % page) for dd in range(d)])
            if L > 0:
                out[i, h] = attend_rows([q[i, h].tolist()], krows, vrows, scale)[0]
    res = dict(query=q, key_cache=kc, value_cache=vc, block_tables=tables,
               context_lens=np.array(lens, dtype=np.int32), out=out)
    if fp8:
        res.update(k_scale=ks, v_scale=vs)
    return res


def case_mx(rng, b, h, s, d, causal):
    finite = [c for c in range(256) if (c & 0x7F) != 0x7F]
    codes = {n: rng.choice(finite, size=(b, h, s, d)).astype(np.uint8) for n in "qkv"}
    scales = {n: rng.integers(120, 131, size=(b, h, s, d // 32)).astype(np.uint8) for n in "qkv"}

    def deq(n, i, hh, t):
        return [e4m3_value(int(codes[n][i, hh, t, dd])) * 2.0 ** (int(scales[n][i, hh, t, dd // 32]) - 127)
                for dd in range(d)]
    scale = 1.0 / math.sqrt(d)
    out = np.zeros((b, h, s, d))
    for i in range(b):
        for hh in range(h):
            qr = [deq("q", i, hh, t) for t in range(s)]
            kr = [deq("k", i, hh, t) for t in range(s)]
            vr = [deq("v", i, hh, t) for t in range(s)]
            out[i, hh] = attend_rows(qr, kr, vr, scale, 0 if causal else None)
    return dict(q=codes["q"], k=codes["k"], v=codes["v"], q_scale=scales["q"],
                k_scale=scales["k"], v_scale=scales["v"], out=out, causal=np.array(causal))


def main():
    rng = np.random.default_rng(0)
    cases = {
        "attn_causal_d64": case_attention(rng, 1, 2, 2, 17, 64, True),
        "attn_full_d64": case_attention(rng, 1, 2, 2, 33, 64, False),
        "attn_gqa_causal_d128": case_attention(rng, 1, 4, 2, 9, 128, True),
        "paged_d64": case_paged(rng, [1, 16, 37, 0], 4, 2, 64, fp8=False),
        "fp8_paged_d128": case_paged(rng, [5, 16, 33], 4, 1, 128, fp8=True),
        "mx_causal": case_mx(rng, 1, 1, 9, 128, True),
    }
    flat = {}
    for cname, arrays in cases.items():
        for k, v in arrays.items():
            flat[f"{cname}/{k}"] = v
    np.savez_compressed(OUT, **flat)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(cases)} cases)")


if __name__ == "__main__":
    main()
