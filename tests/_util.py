"""Shared test helpers: tolerances, input builders, oracle adapters."""
import math

import numpy as np
import torch

import oracle

# north_star tolerances against the fp32 oracle
TOL_16BIT = dict(max_abs=2e-2, mean_abs=2e-3)
TOL_FP8 = dict(max_abs=5e-2, mean_abs=None)


def to_np(t):
    return t.detach().float().cpu().numpy()


def assert_close(out, ref, max_abs, mean_abs=None, name=""):
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert out.shape == ref.shape, f"{name}: shape {out.shape} != {ref.shape}"
    assert np.isfinite(out).all(), f"{name}: non-finite values in output"
    err = np.abs(out - ref)
    mx = float(err.max()) if err.size else 0.0
    mean = float(err.mean()) if err.size else 0.0
    assert mx <= max_abs, f"{name}: max abs error {mx:.3e} > {max_abs}"
    if mean_abs is not None:
        assert mean <= mean_abs, f"{name}: mean abs error {mean:.3e} > {mean_abs}"
    return mx, mean


def qkv(b, hq, s, d, dtype, device, hkv=None, gen=None):
    hkv = hkv or hq
    q = torch.randn(b, hq, s, d, device=device, generator=gen).to(dtype)
    k = torch.randn(b, hkv, s, d, device=device, generator=gen).to(dtype)
    v = torch.randn(b, hkv, s, d, device=device, generator=gen).to(dtype)
    return q, k, v


def build_paged(lens, hq, hkv, d, dtype, device, fp8=False, per_block=True, pool=None,
                page=16, seed=0):
    """Paged GQA decode inputs in the reference layout [blocks, Hkv, D, page].

    A pool of ``pool`` pages (default: exactly the pages needed) ~N(0,1) is
    made on ``device``; sequence n gets the next ceil(L_n/16) entries of a
    random permutation of the pool (tests/_utils.py:105-133 generalised to a
    shared pool and GQA). FP8: per-(page, kv-head) scale amax/448 (or one per
    kv head if ``per_block`` is False) and e4m3 codes (tests/test_kernels_misc.py:52-55).
    """
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    n = len(lens)
    pages = [(int(L) + page - 1) // page for L in lens]
    need = sum(pages)
    pool = max(pool or need, need, 1)
    max_blocks = max(pages + [1])
    perm = torch.randperm(pool, device=device, generator=g).to(torch.int32)
    tables = torch.zeros((n, max_blocks), dtype=torch.int32, device=device)
    cur = 0
    for i, p in enumerate(pages):
        if p:
            tables[i, :p] = perm[cur:cur + p]
        cur += p
    q = torch.randn(n, hq, d, device=device, generator=g).to(dtype)
    kf = torch.randn(pool, hkv, d, page, device=device, generator=g)
    vf = torch.randn(pool, hkv, d, page, device=device, generator=g)
    case = dict(query=q, block_tables=tables,
                context_lens=torch.tensor(lens, dtype=torch.int32, device=device))
    if not fp8:
        case.update(key_cache=kf.to(dtype), value_cache=vf.to(dtype))
    else:
        if per_block:
            ks = (kf.abs().amax(dim=(2, 3)) / 448.0).clamp_min(1e-8)
            vs = (vf.abs().amax(dim=(2, 3)) / 448.0).clamp_min(1e-8)
            k8 = (kf / ks[:, :, None, None]).to(torch.float8_e4m3fn)
            v8 = (vf / vs[:, :, None, None]).to(torch.float8_e4m3fn)
        else:
            ks = (kf.abs().amax(dim=(0, 2, 3)) / 448.0).clamp_min(1e-8)
            vs = (vf.abs().amax(dim=(0, 2, 3)) / 448.0).clamp_min(1e-8)
            k8 = (kf / ks[None, :, None, None]).to(torch.float8_e4m3fn)
            v8 = (vf / vs[None, :, None, None]).to(torch.float8_e4m3fn)
        case.update(key_cache=k8.view(torch.uint8), value_cache=v8.view(torch.uint8),
                    k_scale=ks.float().contiguous(), v_scale=vs.float().contiguous())
    del kf, vf
    return case


def paged_oracle(case, seqs=None, dtype=np.float32):
    """Oracle output [len(seqs), Hq, D] for the selected sequences, copying
    only their pages to the host (arithmetic in `dtype`)."""
    n = case["query"].shape[0]
    seqs = list(range(n)) if seqs is None else list(seqs)
    lens = case["context_lens"].cpu().numpy()
    tables = case["block_tables"].cpu().numpy()
    page = case["key_cache"].shape[-1]
    ids, sub_tables = [], np.zeros((len(seqs), tables.shape[1]), dtype=np.int64)
    for j, i in enumerate(seqs):
        nb = (int(lens[i]) + page - 1) // page
        for b in range(nb):
            sub_tables[j, b] = len(ids)
            ids.append(int(tables[i, b]))
    idx = torch.tensor(ids if ids else [0], dtype=torch.long, device=case["key_cache"].device)
    kc = case["key_cache"].index_select(0, idx)
    vc = case["value_cache"].index_select(0, idx)
    fp8 = "k_scale" in case
    if fp8:
        kc_np, vc_np = kc.cpu().numpy(), vc.cpu().numpy()
        if case["k_scale"].dim() == 2:
            ks = case["k_scale"].index_select(0, idx).cpu().numpy()
            vs = case["v_scale"].index_select(0, idx).cpu().numpy()
        else:
            ks, vs = case["k_scale"].cpu().numpy(), case["v_scale"].cpu().numpy()
    else:
        kc_np, vc_np, ks, vs = to_np(kc), to_np(vc), None, None
    q = to_np(case["query"])[seqs]
    return oracle.paged_decode(q, kc_np, vc_np, sub_tables, lens[seqs],
                               k_scale=ks, v_scale=vs, dtype=dtype)


def mx_inputs(b, h, s, d, device, seed=0):
    """C5-style MXFP8 inputs: x = N(0,1) * U(0.5, 4), OCP MX e4m3 + e8m0 per 32."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    out = {}
    for name in ("q", "k", "v"):
        x = (torch.randn(b, h, s, d, generator=g) * torch.empty(b, h, s, d).uniform_(0.5, 4, generator=g))
        codes, sc = oracle.mx_quantize(x.numpy())
        out[name] = torch.from_numpy(codes).to(device)
        out[name + "_scale"] = torch.from_numpy(sc).to(device)
    return out


def default_scale(d):
    return 1.0 / math.sqrt(d)


def balanced_walk_taken(n, hq, hkv, d, max_blocks, fp8):
    """Whether a paged decode launch of these sizes takes the balanced
    (stream-K) walk of decode.hip (paged_plan there): more than one split of
    the longest context, at most 1024 sequences, and the walk's partials (one
    wave per SIMD, two rows of min(16, Hq/Hkv) heads per wave, plus the
    sequences' prefix) within the workspace every caller provides
    (N * Hq * ceil(max_blocks / 64) rows of D + 1 floats)."""
    split_pages = 128 if fp8 else 64
    grid = 4 * torch.cuda.get_device_properties(0).multi_processor_count
    sk = 2 * grid * min(16, hq // hkv) * (d + 1) * 4 + 4 * n
    contract = n * hq * (-(-max_blocks // 64)) * (d + 1) * 4
    return max_blocks > split_pages and n <= 1024 and sk <= contract
