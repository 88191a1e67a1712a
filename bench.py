#!/usr/bin/env python3
"""Benchmark of the attention forward hot path on one MI355X.

Headline (BASELINE.json metric, config C2): bf16 causal prefill, q/k/v ~ N(0,1)
[4, 32, 4096, 128], fp32 accumulate, bf16 out, inputs resident in HBM. A step
is one ``cuda_llm.flash_attention`` call; FLOPs per step follow the
reference's convention 2*B*H*S^2*D for causal, 4*B*H*S^2*D otherwise
(benchmark_pytorch.py:115-117).

The same JSON line carries, under "fp8_decode", the metric's second half:
FP8 paged GQA decode at C4 (N=256, Hq=32/Hkv=8, D=128, L ~ U[2048, 32768],
e4m3 cache with per-(page, kv-head) fp32 scales). Its algorithmic bytes are
the K/V codes of the context tokens, the scales of the pages read, q, out and
the block-table entries. "extra" holds the other BASELINE configs (C2'
non-causal prefill, C3 bf16 paged decode, C5 MXFP8) and a plain copy used to
calibrate HBM counters. Decode lines also carry the measured streaming-read
ceiling (``ca_stream_read`` over a 4 GiB buffer) as "measured_read_peak".

Timing: W untimed warm-up steps, then K steps between HIP events recorded on
the stream the kernels run on (torch's current stream), bracketed by device
synchronisation. ``cpu_baseline`` times the numpy oracle on a bounded sample
of the same inputs on this host's cores (a reported baseline only).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
                       [--workload all|prefill|prefill_nc|decode_fp8|decode_bf16|mxfp8|backward|copy|read|refgrid|host]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16/fp16 MFMA (published)
PEAK_FP8_TFLOPS = 5000.0    # MI355X dense fp8 / MXFP8 MFMA (published)
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E (published)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# Minimum GPU-busy time of the warm-up: the GPU needs ~0.1-0.2 s of load to
# reach its sustained clock, so a few warm-up launches (the driver's 5) would
# time the first steps at a ramping clock. The warm-up runs at least `warmup`
# launches and keeps launching until this much time has passed.
WARM_SECONDS = 0.25
WARM_LOG = {}  # workload label -> {"launches": n, "seconds": s} of its last warm-up


def time_steps(fn, steps, warmup, label=None):
    """ms per step of `fn` over `steps` launches between HIP events on the
    current stream, after a warm-up of at least `warmup` launches and at least
    WARM_SECONDS of wall time (recorded in WARM_LOG[label])."""
    import torch
    t0 = time.perf_counter()
    n = 0
    for _ in range(warmup):
        fn()
        n += 1
    torch.cuda.synchronize()
    while time.perf_counter() - t0 < WARM_SECONDS:
        for _ in range(4):
            fn()
            n += 1
        torch.cuda.synchronize()
    if label:
        WARM_LOG[label] = {"launches": n, "seconds": round(time.perf_counter() - t0, 3)}
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per step


def _stream_reader(nbytes):
    """A call that streams `nbytes` of a resident buffer through ca_stream_read."""
    import ctypes
    import torch
    from cuda_amd import _lib
    x = torch.empty(nbytes // 4, dtype=torch.int32, device="cuda").random_(generator=_gen())
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return lambda: _lib.call("ca_stream_read", ctypes.c_void_p(x.data_ptr()), nbytes,
                             ctypes.c_void_p(sink.data_ptr()), st)


def time_cold(fn, reps=20, flush_bytes=1 << 30):
    """Median ms of one call of `fn` issued right after a pass over a 1 GiB
    buffer (read and written by a torch kernel, so kernel traces keep this
    library's kernels apart), which leaves none of fn's inputs in the L2s or
    the 256 MB MALL."""
    import torch
    buf = torch.zeros(flush_bytes // 4, dtype=torch.int32, device="cuda")
    flush = lambda: buf.add_(1)
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps)]
    torch.cuda.synchronize()
    for e0, e1 in ev:
        flush()
        e0.record(stream)
        fn()
        e1.record(stream)
    torch.cuda.synchronize()
    t = sorted(e0.elapsed_time(e1) for e0, e1 in ev)
    return t[len(t) // 2]


def _traffic(key):
    """HBM bytes per step measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE of every kernel of the step, scaled by the copy-kernel
    calibration), committed in profiles/traffic.json by --traffic-json."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        return float(t[key]["fetch_bytes"]) + float(t[key]["write_bytes"])
    except (OSError, KeyError, ValueError, TypeError):
        return None


def blas_threads():
    try:
        from threadpoolctl import threadpool_info
        n = [i.get("num_threads", 0) for i in threadpool_info() if i.get("user_api") == "blas"]
        return max(n) if n else os.cpu_count()
    except Exception:
        return os.cpu_count()


def host_info():
    """CPU model and counts of this host, reported beside every CPU figure."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count()
    return {"cpu_model": model, "host_cpus": os.cpu_count(), "cpus_available": avail}


def _gen(seed=0):
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return g


# ---------------------------------------------------------------------------
# workloads: each returns dict(ms, value, unit, bound, peak, state...)
# ---------------------------------------------------------------------------
# --no-cold: skip the cold-cache timing (profiling runs, whose summaries take
# the last `steps` dispatches of each kernel as the timed ones)
SKIP_COLD = False


def w_prefill(steps, warmup, causal=True, B=4, H=32, S=4096, D=128):
    import torch
    import cuda_llm
    g = _gen()
    q, k, v = (torch.randn(B, H, S, D, device="cuda", generator=g).to(torch.bfloat16) for _ in range(3))
    fn = lambda: cuda_llm.flash_attention(q, k, v, is_causal=causal)
    ms = time_steps(fn, steps, warmup, "prefill" if causal else "prefill_nc")
    flops = (2.0 if causal else 4.0) * B * H * S * S * D
    tf = flops / (ms * 1e-3) / 1e12
    cold = None if SKIP_COLD else time_cold(fn)
    return dict(ms=ms, value=tf, unit="TFLOP/s", bound="mfma", peak=PEAK_BF16_TFLOPS,
                work=flops, qkv=(q, k, v), causal=causal,
                cold=None if cold is None else
                {"ms_per_step": round(cold, 4), "value": round(flops / (cold * 1e-3) / 1e12, 2),
                 "note": "median of 20 single calls, each after a pass over a 1 GiB buffer"},
                config={"workload": f"C2{'' if causal else chr(39)} bf16 {'causal' if causal else 'non-causal'} prefill (flash_attention)",
                        "batch": B, "heads": H, "seq_len": S, "head_dim": D, "causal": causal})


def w_backward(steps, warmup, causal=True, B=4, H=32, S=4096, D=128):
    """Backward of the C2 prefill (dq, dk, dv from q, k, v, out, dout, lse).
    Work: five S x S x D products per (b, h) (S, dP, dV, dK, dQ), 2.5x the
    forward's FLOP count, halved when causal (the same convention)."""
    import torch
    import cuda_llm
    g = _gen()
    q, k, v, dout = (torch.randn(B, H, S, D, device="cuda", generator=g).to(torch.bfloat16)
                     for _ in range(4))
    out, lse = cuda_llm.flash_attention_forward_lse(q, k, v, is_causal=causal)
    ms = time_steps(lambda: cuda_llm.flash_attention_backward(dout, q, k, v, out, lse,
                                                              is_causal=causal), steps, warmup,
                    "backward")
    flops = 2.5 * (2.0 if causal else 4.0) * B * H * S * S * D
    tf = flops / (ms * 1e-3) / 1e12
    return dict(ms=ms, value=tf, unit="TFLOP/s", bound="mfma", peak=PEAK_BF16_TFLOPS, work=flops,
                config={"workload": f"C2 bf16 {'causal' if causal else 'non-causal'} prefill backward "
                                    "(flash_attention_backward)",
                        "batch": B, "heads": H, "seq_len": S, "head_dim": D, "causal": causal})


def cpu_prefill(r, seconds):
    """Oracle (numpy fp32) on as many (b, h) heads of the same inputs as fit in
    ~``seconds``; heads are independent, so the rate scales exactly."""
    import oracle
    q, k, v = r["qkv"]
    B, H, S, D = q.shape
    done, el = 0, 0.0  # oracle time only; device->host copies excluded
    for b in range(B):
        for h in range(H):
            qq, kk, vv = (t[b:b + 1, h:h + 1].float().cpu().numpy() for t in (q, k, v))
            t1 = time.perf_counter()
            oracle.attention(qq, kk, vv, is_causal=r["causal"])
            el += time.perf_counter() - t1
            done += 1
            if el >= seconds:
                break
        if el >= seconds:
            break
    flops = (2.0 if r["causal"] else 4.0) * S * S * D * done
    return dict(value=flops / el / 1e12, unit="TFLOP/s", cores=blas_threads(), kind="port",
                sample=f"{done} of {B * H} (b,h) heads of the same inputs, numpy fp32 oracle "
                       f"(oracle/attention.py), {el:.1f} s", **host_info())


def make_paged(N, Hq, Hkv, D, lens, fp8, pool=None, seed=0):
    import torch
    pages = (lens + 15) // 16
    need = int(pages.sum())
    P = max(pool or need, need)
    dev = torch.device("cuda")
    g = _gen(seed)
    perm = torch.randperm(P, device=dev, generator=g).to(torch.int32)
    max_blocks = int(pages.max())
    tables = torch.zeros(N, max_blocks, dtype=torch.int32, device=dev)
    starts = torch.cumsum(pages, 0) - pages
    for i in range(N):
        tables[i, :int(pages[i])] = perm[int(starts[i]):int(starts[i]) + int(pages[i])]
    case = dict(tables=tables, lens=lens.to(torch.int32).to(dev), lens_host=lens.tolist(), P=P)
    chunk = 32768
    if fp8:
        kc = torch.empty(P, Hkv, D, 16, dtype=torch.uint8, device=dev)
        vc = torch.empty_like(kc)
        ks = torch.empty(P, Hkv, dtype=torch.float32, device=dev)
        vs = torch.empty_like(ks)
        for c0 in range(0, P, chunk):
            c1 = min(P, c0 + chunk)
            for cache, sc in ((kc, ks), (vc, vs)):
                x = torch.randn(c1 - c0, Hkv, D, 16, device=dev, generator=g)
                s = (x.abs().amax(dim=(2, 3)) / 448.0).clamp_min(1e-8)
                cache[c0:c1] = (x / s[:, :, None, None]).to(torch.float8_e4m3fn).view(torch.uint8)
                sc[c0:c1] = s
        case.update(kc=kc, vc=vc, ks=ks, vs=vs)
    else:
        kc = torch.empty(P, Hkv, D, 16, dtype=torch.bfloat16, device=dev)
        vc = torch.empty_like(kc)
        for c0 in range(0, P, chunk):
            c1 = min(P, c0 + chunk)
            kc[c0:c1] = torch.randn(c1 - c0, Hkv, D, 16, device=dev, generator=g).to(torch.bfloat16)
            vc[c0:c1] = torch.randn(c1 - c0, Hkv, D, 16, device=dev, generator=g).to(torch.bfloat16)
        case.update(kc=kc, vc=vc)
    case["query"] = torch.randn(N, Hq, D, device=dev, generator=g).to(torch.bfloat16)
    elem = 1 if fp8 else 2
    case["alg_bytes"] = (int(lens.sum()) * Hkv * D * 2 * elem     # K + V of the context tokens
                         + (need * Hkv * 4 * 2 if fp8 else 0)     # k/v scales of the pages read
                         + 2 * N * Hq * D * 2                     # q in, out
                         + need * 4 + N * 4)                      # block-table entries, lengths
    return case


def w_decode(steps, warmup, fp8):
    import torch
    import cuda_llm
    gc = torch.Generator().manual_seed(0)
    if fp8:   # C4
        N, lens, pool = 256, torch.randint(2048, 32769, (256,), generator=gc), None
    else:     # C3
        N, lens, pool = 64, torch.randint(512, 8193, (64,), generator=gc), 40000
    c = make_paged(N, 32, 8, 128, lens, fp8, pool=pool)
    if fp8:
        fn = lambda: cuda_llm.fp8_paged_attention_forward(c["query"], c["kc"], c["vc"], c["ks"], c["vs"],
                                                          c["tables"], c["lens"])
    else:
        fn = lambda: cuda_llm.paged_attention_forward(c["query"], c["kc"], c["vc"], c["tables"], c["lens"])
    ms = time_steps(fn, steps, warmup, "decode_fp8" if fp8 else "decode_bf16")
    gbs = c["alg_bytes"] / (ms * 1e-3) / 1e9
    name = "C4 FP8 paged GQA decode" if fp8 else "C3 bf16 paged GQA decode"
    return dict(ms=ms, value=gbs, unit="GB/s", bound="hbm", peak=PEAK_HBM_GBS, work=c["alg_bytes"],
                case=c, fp8=fp8,
                config={"workload": name, "num_seqs": N, "q_heads": 32, "kv_heads": 8, "head_dim": 128,
                        "page": 16, "context": "U[2048, 32768]" if fp8 else "U[512, 8192]",
                        "pool_pages": c["P"], "alg_bytes_per_step": c["alg_bytes"]})


def cpu_decode(r, seconds):
    import numpy as np
    import oracle
    c = r["case"]
    done_tokens = done = 0
    el = 0.0
    for i, L in enumerate(c["lens_host"]):
        nb = (L + 15) // 16
        ids = c["tables"][i, :nb].long()
        kc = c["kc"].index_select(0, ids)
        vc = c["vc"].index_select(0, ids)
        if r["fp8"]:
            kc, vc = kc.cpu().numpy(), vc.cpu().numpy()
            ks = c["ks"].index_select(0, ids).cpu().numpy()
            vs = c["vs"].index_select(0, ids).cpu().numpy()
        else:
            kc, vc = kc.float().cpu().numpy(), vc.float().cpu().numpy()
            ks = vs = None
        q = c["query"][i:i + 1].float().cpu().numpy()
        t1 = time.perf_counter()
        oracle.paged_decode(q, kc, vc, np.arange(nb)[None], [L], k_scale=ks, v_scale=vs)
        el += time.perf_counter() - t1
        done_tokens += L
        done += 1
        if el >= seconds:
            break
    bytes_per_token = c["alg_bytes"] / sum(c["lens_host"])
    return dict(value=done_tokens * bytes_per_token / el / 1e9, unit="GB/s", cores=blas_threads(),
                kind="port", sample=f"{done} of {len(c['lens_host'])} sequences of the same inputs, "
                                    f"numpy oracle (oracle/paged.py), {el:.1f} s", **host_info())


def w_mxfp8(steps, warmup, B=1, H=16, S=8192, D=128):
    import torch
    import cuda_llm
    g = _gen()
    x = {}
    for n in "qkv":
        v = torch.randn(B, H, S, D, device="cuda", generator=g) * \
            torch.empty(B, H, S, D, device="cuda").uniform_(0.5, 4, generator=g)
        blk = v.view(B, H, S, D // 32, 32)
        amax = blk.abs().amax(-1)
        e = torch.floor(torch.log2(amax)) - 8
        sc = torch.ldexp(torch.ones_like(e), e.to(torch.int32))
        x[n] = (blk / sc[..., None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(B, H, S, D)
        x[n + "s"] = (e + 127).to(torch.uint8)
    fn = lambda: cuda_llm.fused_microscaled_attention(x["q"], x["qs"], x["k"], x["ks"], x["v"], x["vs"],
                                                      is_causal=True)
    ms = time_steps(fn, steps, warmup, "mxfp8")
    flops = 2.0 * B * H * S * S * D
    return dict(ms=ms, value=flops / (ms * 1e-3) / 1e12, unit="TFLOP/s", bound="mfma",
                peak=PEAK_FP8_TFLOPS, work=flops,
                config={"workload": "C5 MXFP8 causal attention", "batch": B, "heads": H, "seq_len": S,
                        "head_dim": D, "note": "QK on fp8 scaled MFMA, PV on bf16 MFMA"})


def w_c1(steps, warmup, B=2, H=8, S=1024, D=64):
    """C1 (the workload of the reference's ref_attention,
    tests/_utils.py:48-53): fp32 q, k, v ~ N(0,1) [2, 8, 1024, 64], causal,
    scale 1/8. The oracle (numpy fp32) runs the whole config on this host's
    cores, and the fp32 HIP prefill runs it on the GPU; both are checked
    against each other (max-abs 1e-4, the reference's float32 tolerance)."""
    import numpy as np
    import torch
    import cuda_llm
    import oracle
    g = _gen()
    q, k, v = (torch.randn(B, H, S, D, device="cuda", generator=g) for _ in range(3))
    fn = lambda: cuda_llm.flash_attention(q, k, v, is_causal=True)
    ms = time_steps(fn, steps, warmup, "c1")
    flops = 2.0 * B * H * S * S * D
    qn, kn, vn = (t.cpu().numpy() for t in (q, k, v))
    reps, el = 0, 0.0
    while el < 2.0 or reps < 3:
        t1 = time.perf_counter()
        ref = oracle.attention(qn, kn, vn, is_causal=True)
        el += time.perf_counter() - t1
        reps += 1
    err = float(np.abs(fn().cpu().numpy() - ref).max())
    return dict(ms=ms, value=flops / (ms * 1e-3) / 1e12, unit="TFLOP/s", bound="mfma",
                peak=157.3, work=flops, max_abs_err_vs_oracle=err,
                cpu={"value": flops * reps / el / 1e12, "unit": "TFLOP/s", "cores": blas_threads(),
                     "kind": "port", "sample": f"the whole config, {reps} runs of the numpy fp32 "
                                               f"oracle (oracle/attention.py), {el:.1f} s",
                     **host_info()},
                config={"workload": "C1 fp32 causal prefill (flash_attention)", "batch": B,
                        "heads": H, "seq_len": S, "head_dim": D, "causal": True,
                        "note": "GPU: fp32 prefill on v_mfma_f32_32x32x2_f32, priced against the "
                                "fp32 MFMA peak 157.3 TFLOP/s"})


def w_copy(steps, warmup, nbytes=2 << 30):
    import torch
    x = torch.empty(nbytes // 2, dtype=torch.bfloat16, device="cuda").normal_()
    y = torch.empty_like(x)
    ms = time_steps(lambda: y.copy_(x), steps, warmup, "copy")
    return dict(ms=ms, value=2 * nbytes / (ms * 1e-3) / 1e9, unit="GB/s", bound="hbm",
                peak=PEAK_HBM_GBS, work=2 * nbytes,
                config={"workload": "device copy (HBM counter calibration)", "bytes": nbytes})


def w_read(steps, warmup, nbytes=4 << 30):
    """Streaming-read ceiling: ca_stream_read over a resident buffer (the
    measured second denominator of the HBM-bound decode lines)."""
    ms = time_steps(_stream_reader(nbytes), steps, warmup, "read")
    return dict(ms=ms, value=nbytes / (ms * 1e-3) / 1e9, unit="GB/s", bound="hbm",
                peak=PEAK_HBM_GBS, work=nbytes,
                config={"workload": "streaming read (measured HBM read ceiling)", "bytes": nbytes})


def _sdpa_ms(q, k, v, causal, steps, warmup):
    """torch's own scaled_dot_product_attention on the same inputs, flash
    backend only (no math fallback); None where torch has no such kernel."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    gqa = q.shape[1] != k.shape[1]
    try:
        with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
            return time_steps(lambda: F.scaled_dot_product_attention(q, k, v, is_causal=causal,
                                                                      enable_gqa=gqa),
                              steps, warmup)
    except RuntimeError as e:
        log(f"torch sdpa (flash) unavailable: {str(e).splitlines()[0][:120]}")
        return None


def w_refgrid(steps, warmup):
    """The reference benchmark's own grid (benchmark_pytorch.py:627-658): fp16,
    head dim 64, its shapes, table layouts and units (prefill TFLOP/s with
    2 (causal) or 4 x B H S^2 D, backward 10 B H S^2 D, decode GB/s of K + V
    bytes N H L D elem 2), run on this build's entry points. Prefill lines
    also time torch's flash SDPA on the same inputs. The C2 shape closes the
    grid for the same comparison at head dim 128. Not part of the default run."""
    import torch
    import cuda_llm
    st, wu = min(steps, 100), min(warmup, 50)
    f16 = torch.float16
    g = _gen()
    rows = []

    def randn(*shape, dtype=f16):
        return torch.randn(*shape, device="cuda", generator=g).to(dtype)

    def add(name, ref, ms, work, unit, sdpa=None, **shape):
        val = work / (ms * 1e-3) / (1e12 if unit == "TFLOP/s" else 1e9)
        row = {"case": name, "ref": ref, **shape, "ms": round(ms, 4), "value": round(val, 2),
               "unit": unit}
        if sdpa is not None:
            row["torch_sdpa_ms"] = round(sdpa, 4)
            row["speedup_vs_torch_sdpa"] = round(sdpa / ms, 2)
        rows.append(row)
        log(f"{name} {shape}: {ms:.4f} ms, {val:.1f} {unit}"
            + (f", torch sdpa {sdpa:.4f} ms" if sdpa else ""))

    def prefill(name, ref, fn, B, Hq, Hkv, S, D, causal, dtype=f16, rope=False):
        q, k, v = randn(B, Hq, S, D, dtype=dtype), randn(B, Hkv, S, D, dtype=dtype), \
            randn(B, Hkv, S, D, dtype=dtype)
        if rope:
            inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, device="cuda").float() / D))
            fr = torch.outer(torch.arange(S, device="cuda").float(), inv)
            emb = torch.cat((fr, fr), -1)
            cs, sn = emb.cos().contiguous(), emb.sin().contiguous()
            ms = time_steps(lambda: fn(q, k, v, cs, sn, is_causal=causal), st, wu)
            sd = None
        else:
            ms = time_steps(lambda: fn(q, k, v, is_causal=causal), st, wu)
            sd = _sdpa_ms(q, k, v, causal, st, wu)
        add(name, ref, ms, (2.0 if causal else 4.0) * B * Hq * S * S * D, "TFLOP/s", sd,
            B=B, Hq=Hq, Hkv=Hkv, S=S, D=D, causal=causal, dtype=str(dtype).split(".")[-1])
        del q, k, v

    for S in (2048, 4096, 8192):
        prefill("flash_attention_forward", "benchmark_pytorch.py:636-637",
                cuda_llm.flash_attention_forward, 2, 32, 32, S, 64, True)
    for N in (32, 64, 128):
        nb = 2048 // 16
        q = randn(N, 32, 64)
        kc, vc = randn(N * nb, 32, 64, 16), randn(N * nb, 32, 64, 16)
        tab = torch.arange(N * nb, device="cuda", dtype=torch.int32).view(N, nb)
        lens = torch.full((N,), 2048, device="cuda", dtype=torch.int32)
        ms = time_steps(lambda: cuda_llm.paged_attention_forward(q, kc, vc, tab, lens), st, wu)
        add("paged_attention_forward", "benchmark_pytorch.py:639-641", ms, N * 32 * 2048 * 64 * 2 * 2,
            "GB/s", N=N, H=32, D=64, context=2048)
        del q, kc, vc
    for N in (32, 64, 128):
        nb = 4096 // 16
        q = randn(N, 32, 64)
        # valid e4m3 bytes (0x7f / 0xff are NaN codes), per-(page, head) scale 0.01
        codes = lambda: (torch.randint(0, 255, (N * nb, 32, 64, 16), device="cuda", generator=g,
                                       dtype=torch.int32) % 127
                         + 128 * torch.randint(0, 2, (N * nb, 32, 64, 16), device="cuda",
                                               generator=g, dtype=torch.int32)).to(torch.uint8)
        kc, vc = codes(), codes()
        sc = torch.full((N * nb, 32), 0.01, device="cuda")
        tab = torch.arange(N * nb, device="cuda", dtype=torch.int32).view(N, nb)
        lens = torch.full((N,), 4096, device="cuda", dtype=torch.int32)
        ms = time_steps(lambda: cuda_llm.fp8_paged_attention_forward(q, kc, vc, sc, sc, tab, lens),
                        st, wu)
        add("fp8_paged_attention_forward", "benchmark_pytorch.py:643-645", ms,
            N * 32 * 4096 * 64 * 1 * 2, "GB/s", N=N, H=32, D=64, context=4096)
        del q, kc, vc
    for S in (2048, 4096):
        prefill("fused_rope_flash_attention", "benchmark_pytorch.py:647-649",
                cuda_llm.fused_rope_flash_attention, 2, 32, 32, S, 64, True, rope=True)
    for S in (2048, 4096, 8192):
        prefill("fused_gqa_forward", "benchmark_pytorch.py:651-653",
                cuda_llm.fused_gqa_forward, 2, 32, 8, S, 64, True)
    for S in (4096, 8192, 16384):
        q, k, v = randn(8, 32, 1, 64), randn(8, 32, S, 64), randn(8, 32, S, 64)
        ms = time_steps(lambda: cuda_llm.async_flash_decode(q, k, v), st, wu)
        add("async_flash_decode", "benchmark_pytorch.py:655-657", ms, 8 * 32 * S * 64 * 2 * 2,
            "GB/s", B=8, H=32, S_kv=S, D=64)
        del q, k, v
    for S in (2048, 4096):
        q, k, v, do = (randn(2, 32, S, 64) for _ in range(4))
        o, lse = cuda_llm.flash_attention_forward_lse(q, k, v, is_causal=False)
        ms = time_steps(lambda: cuda_llm.flash_attention_backward(do, q, k, v, o, lse,
                                                                  is_causal=False), st, wu)
        add("flash_attention_backward", "benchmark_pytorch.py:659-661", ms,
            10.0 * 2 * 32 * S * S * 64, "TFLOP/s", B=2, H=32, S=S, D=64, causal=False)
        del q, k, v, do, o, lse
    for S in (4096, 8192, 16384):
        prefill("flash_attention_v3_hopper", "benchmark_pytorch.py:667-669",
                cuda_llm.flash_attention_v3_hopper, 2, 32, 32, S, 64, False)
    prefill("flash_attention (C2)", "BASELINE config C2", cuda_llm.flash_attention, 4, 32, 32, 4096,
            128, True, dtype=torch.bfloat16)
    torch.cuda.empty_cache()
    return rows


_READ_CEILING = {}


def w_host(steps, warmup):
    """Host cost per call of the entry points on shapes whose kernels take a
    few microseconds, so a loop of calls is bound by the host: the Python
    API (argument checks, output and workspace allocation, ctypes call), the
    C ABI through ctypes with preallocated buffers, and torch's own dispatch
    of one small elementwise op as the yardstick. Microseconds per call
    (wall clock over n calls, one synchronisation at the end)."""
    import ctypes
    import time
    import torch
    import cuda_llm
    import cuda_amd._lib as L
    n = max(200, steps * 10)
    g = _gen()
    rows = []

    def timed(fn):
        for _ in range(min(warmup, 50)):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n * 1e6

    def gpu(fn):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ts = []
        for _ in range(20):
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e3)
        return sorted(ts)[len(ts) // 2]

    bf = torch.bfloat16
    lib = L.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    # prefill: 1 x 1 x 64 x 128
    q, k, v = (torch.randn(1, 1, 64, 128, device="cuda", generator=g).to(bf) for _ in range(3))
    o = torch.empty_like(q)
    args = (L.CA_BF16, p(q), p(k), p(v), p(o), 1, 1, 1, 64, 128, ctypes.c_float(128 ** -0.5), 1,
            stream)
    rows.append({"case": "flash_attention_forward 1x1x64x128 causal",
                 "api_us": round(timed(lambda: cuda_llm.flash_attention_forward(q, k, v, is_causal=True)), 2),
                 "abi_us": round(timed(lambda: lib.ca_flash_attention_fwd(*args)), 2),
                 "gpu_us": round(gpu(lambda: lib.ca_flash_attention_fwd(*args)), 2)})
    # paged decode: 1 sequence, 32 query / 8 kv heads, 16 tokens
    c = make_paged(1, 32, 8, 128, torch.tensor([16]), False)
    kc, vc, tb, ln, qq = c["kc"], c["vc"], c["tables"], c["lens"], c["query"]
    ws_bytes = int(lib.ca_decode_workspace_bytes(1, 32, 128, tb.shape[1] * 16))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(qq)
    pargs = (L.CA_BF16, p(qq), p(kc), p(vc), p(tb), p(ln), p(out), 1, 32, 8, 128, tb.shape[1], 16,
             kc.shape[0], ctypes.c_float(128 ** -0.5), p(ws), ctypes.c_size_t(ws.numel()), stream)
    rows.append({"case": "paged_attention_forward 1 seq x 32/8 heads x 16 tokens",
                 "api_us": round(timed(lambda: cuda_llm.paged_attention_forward(qq, kc, vc, tb, ln)), 2),
                 "abi_us": round(timed(lambda: lib.ca_paged_attention(*pargs)), 2),
                 "gpu_us": round(gpu(lambda: lib.ca_paged_attention(*pargs)), 2)})
    x = torch.zeros(64, device="cuda")
    rows.append({"case": "torch yardstick: x.add_(1) on 64 floats",
                 "api_us": round(timed(lambda: x.add_(1)), 2), "gpu_us": round(gpu(lambda: x.add_(1)), 2)})
    for r in rows:
        log(f"host: {r}")
    return rows


def read_ceiling(steps, warmup):
    """Measured streaming-read GB/s, once per process."""
    import torch
    if "gbs" not in _READ_CEILING:
        r = w_read(min(steps, 50), min(warmup, 20))
        _READ_CEILING["gbs"] = r["value"]
        log(f"read ceiling: {r['value']:.1f} GB/s")
        torch.cuda.empty_cache()
    return _READ_CEILING["gbs"]


WORKLOADS = {
    "prefill": lambda s, w: w_prefill(s, w, causal=True),
    "prefill_nc": lambda s, w: w_prefill(s, w, causal=False, S=2048),
    "decode_fp8": lambda s, w: w_decode(s, w, fp8=True),
    "decode_bf16": lambda s, w: w_decode(s, w, fp8=False),
    "mxfp8": w_mxfp8,
    "backward": w_backward,
    "c1": w_c1,
    "copy": w_copy,
    "read": w_read,
    "refgrid": w_refgrid,
    "host": w_host,
}
# the workloads whose step traffic profiles/traffic.json holds (every kernel
# of the step: decode = split + merge, MXFP8 = prepare + attention, backward =
# row dot + dK/dV + dQ)
TRAFFIC_WORKLOADS = ("prefill", "prefill_nc", "decode_fp8", "decode_bf16", "mxfp8", "backward", "c1")
TRAFFIC_KEY = {w: w for w in TRAFFIC_WORKLOADS}
# kernels a workload's run launches outside its timed step: the streaming-read
# ceiling the decode lines report beside them, the forward that makes the
# backward's inputs
TRAFFIC_NOT_STEP = {"decode_fp8": ("stream_read",), "decode_bf16": ("stream_read",),
                    "backward": ("prefill_",)}


def summary(name, r, read_gbs=None):
    """One result object. For an HBM-bound decode line, `read_gbs` (the
    measured streaming-read ceiling) is reported beside the nominal peak as a
    second denominator."""
    out = {"value": round(r["value"], 2), "unit": r["unit"], "ms_per_step": round(r["ms"], 4),
           "config": r["config"],
           "roofline": {"bound": r["bound"], "achieved": round(r["value"], 2), "peak": r["peak"],
                        "unit": r["unit"], "frac": round(r["value"] / r["peak"], 4),
                        "traffic": _traffic(TRAFFIC_KEY.get(name, name))}}
    if r.get("cold"):
        out["cold"] = r["cold"]
    if name in WARM_LOG:
        out["warmup_run"] = WARM_LOG[name]
    if "cpu" in r:
        out["cpu_baseline"] = r["cpu"]
    if "max_abs_err_vs_oracle" in r:
        out["max_abs_err_vs_oracle"] = r["max_abs_err_vs_oracle"]
    if read_gbs:
        out["roofline"]["measured_read_peak"] = round(read_gbs, 2)
        out["roofline"]["frac_of_measured"] = round(r["value"] / read_gbs, 4)
    return out


# ---------------------------------------------------------------------------
# profile summaries (rocprofv3 CSV output of a bench.py run -> text)
# ---------------------------------------------------------------------------
def _kernel_short_name(name):
    """'void ca::foo<...>(args)' -> 'ca::foo<...>'."""
    n = name[5:] if name.startswith("void ") else name
    n = n.replace("(anonymous namespace)::", "")
    depth = 0
    for i, ch in enumerate(n):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return n[:i]
    return n


def trace_summary(path, last):
    """Per-kernel durations from a rocprofv3 --kernel-trace CSV over the last
    `last` dispatches of each of this library's kernels: in a bench.py run of
    one workload with --no-cold those are the timed launches (the warm-up
    launches come first), so the averages are comparable with the run's
    ms_per_step. Prints one markdown table."""
    import csv
    by = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            name = _kernel_short_name(r["Kernel_Name"])
            if name.startswith("ca::"):
                by.setdefault(name, []).append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    print("| kernel | dispatches | timed (last) | avg µs | median µs | min µs | max µs |")
    print("|---|---|---|---|---|---|---|")
    for name, ts in sorted(by.items(), key=lambda kv: kv[1][0][0]):
        ts.sort()
        d = sorted((e - s) / 1e3 for s, e in ts[-last:])
        print(f"| `{name}` | {len(ts)} | {len(d)} | {sum(d) / len(d):.1f} | {d[len(d) // 2]:.1f} | "
              f"{d[0]:.1f} | {d[-1]:.1f} |")


def pmc_summary(path):
    """Per-kernel averages of every counter of a rocprofv3 --pmc CSV (this
    library's kernels only), printed as one JSON object."""
    import csv
    acc = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            name = _kernel_short_name(r["Kernel_Name"])
            if name.startswith("ca::") or "copyBuffer" in name:
                c = acc.setdefault(name, {}).setdefault(r["Counter_Name"], [0.0, 0])
                c[0] += float(r["Counter_Value"])
                c[1] += 1
    print(json.dumps({k: {c: v[0] / v[1] for c, v in d.items()} for k, d in acc.items()}, indent=1))


def _pmc_means(path, counter):
    """{kernel: mean counter value per dispatch} of this library's kernels
    (and the copy kernel) in one rocprofv3 --pmc CSV."""
    import csv
    acc = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            name = _kernel_short_name(r["Kernel_Name"])
            if r["Counter_Name"] == counter and (name.startswith("ca::") or "copyBuffer" in name):
                a = acc.setdefault(name, [0.0, 0])
                a[0] += float(r["Counter_Value"])
                a[1] += 1
    return {k: v[0] / v[1] for k, v in acc.items()}


def traffic_json(pmc_dir, out):
    """Writes the step traffic of each TRAFFIC_WORKLOADS workload from one
    FETCH_SIZE and one WRITE_SIZE run per workload (rocprofv3 -d
    <pmc_dir>/<workload>_fetch, _write; and copy_fetch, copy_write for the
    calibration): per kernel the mean KiB per dispatch, summed over the
    step's kernels (each runs once per step), scaled to bytes by what the
    counters read for the copy of w_copy's known size."""
    csvp = lambda w, c: os.path.join(pmc_dir, f"{w}_{c}", "run_counter_collection.csv")
    nbytes = 2 << 30
    cf = _pmc_means(csvp("copy", "fetch"), "FETCH_SIZE")
    cw = _pmc_means(csvp("copy", "write"), "WRITE_SIZE")
    kf = max(cf.values()) * 1024
    kw = max(cw.values()) * 1024
    res = {"_calibration": {"kernel": next(iter(cf)), "bytes_read": nbytes, "bytes_written": nbytes,
                            "fetch_size_kib": kf / 1024, "write_size_kib": kw / 1024,
                            "fetch_factor": nbytes / kf, "write_factor": nbytes / kw}}
    for w in TRAFFIC_WORKLOADS:
        f = _pmc_means(csvp(w, "fetch"), "FETCH_SIZE")
        wr = _pmc_means(csvp(w, "write"), "WRITE_SIZE")
        skip = ("copyBuffer",) + TRAFFIC_NOT_STEP.get(w, ())
        ks = sorted(k for k in set(f) & set(wr) if not any(x in k for x in skip))
        res[w] = {"kernels": ks,
                  "fetch_bytes": round(sum(f[k] for k in ks) * 1024 * nbytes / kf),
                  "write_bytes": round(sum(wr[k] for k in ks) * 1024 * nbytes / kw)}
    with open(out, "w") as fh:
        json.dump(res, fh, indent=1)
        fh.write("\n")
    print(json.dumps(res, indent=1))


def main():
    ap = argparse.ArgumentParser(description="attention forward hot path benchmark (one MI355X)")
    ap.add_argument("--gpus", type=int, default=1)
    # 200 warm-up launches (0.1-0.3 s) bring the GPU to its sustained clock;
    # with a handful the first timed launches still run at a ramping clock
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--workload", default="all", choices=["all"] + list(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cold", action="store_true",
                    help="skip the cold-cache prefill timing (profiling runs)")
    ap.add_argument("--trace-summary", metavar="CSV",
                    help="summarise a rocprofv3 kernel-trace CSV over each kernel's last --steps "
                         "dispatches (no GPU needed)")
    ap.add_argument("--pmc-summary", metavar="CSV",
                    help="average a rocprofv3 --pmc CSV per kernel (no GPU needed)")
    ap.add_argument("--traffic-json", nargs=2, metavar=("PMC_DIR", "OUT"),
                    help="write per-workload step traffic from FETCH_SIZE / WRITE_SIZE runs "
                         "(no GPU needed)")
    args = ap.parse_args()
    if args.traffic_json:
        traffic_json(*args.traffic_json)
        return
    if args.trace_summary:
        trace_summary(args.trace_summary, args.steps)
        return
    if args.pmc_summary:
        pmc_summary(args.pmc_summary)
        return
    global SKIP_COLD
    SKIP_COLD = args.no_cold
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (--gpus {args.gpus} "
              "requested). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    props = torch.cuda.get_device_properties(0)

    if args.workload == "refgrid":
        rows = w_refgrid(args.steps, args.warmup)
        print(json.dumps({"metric": "reference benchmark grid (benchmark_pytorch.py)", "n_gpus": 1,
                          "data": "synthetic, seeded", "device": props.name, "rows": rows}),
              flush=True)
        return
    if args.workload == "host":
        rows = w_host(args.steps, args.warmup)
        print(json.dumps({"metric": "host microseconds per call (launch-bound shapes)", "n_gpus": 1,
                          "data": "synthetic, seeded", "device": props.name, "rows": rows}),
              flush=True)
        return
    head = "prefill" if args.workload == "all" else args.workload
    log(f"{head} ...")
    r = WORKLOADS[head](args.steps, args.warmup)
    log(f"{head}: {r['ms']:.4f} ms/step, {r['value']:.1f} {r['unit']}")
    is_decode = head.startswith("decode")
    s = summary(head, r, read_ceiling(args.steps, args.warmup) if is_decode else None)
    line = {
        "metric": {"prefill": "prefill TFLOP/s (bf16 causal, B=4 H=32 S=4096 D=128)",
                   "prefill_nc": "prefill TFLOP/s (bf16 non-causal, B=4 H=32 S=2048 D=128)",
                   "decode_fp8": "FP8 paged GQA decode HBM GB/s (C4)",
                   "decode_bf16": "bf16 paged GQA decode HBM GB/s (C3)",
                   "mxfp8": "MXFP8 causal attention TFLOP/s (C5)",
                   "backward": "prefill backward TFLOP/s (bf16 causal, B=4 H=32 S=4096 D=128)",
                   "copy": "device copy GB/s",
                   "read": "streaming read GB/s",
                   "c1": "prefill TFLOP/s (fp32 causal, B=2 H=8 S=1024 D=64)"}[head],
        "value": s["value"], "unit": s["unit"], "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": s["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": {"prefill": "bf16", "prefill_nc": "bf16", "decode_fp8": "e4m3 KV / bf16 q,out / fp32 softmax",
                  "decode_bf16": "bf16", "mxfp8": "mxfp8 e4m3+e8m0 / bf16 out", "backward": "bf16",
                  "copy": "bf16", "read": "u32", "c1": "f32"}[head],
        "data": "synthetic, seeded (torch generator seed 0), resident in HBM",
        "config": dict(s["config"], parallelism="none (1 GPU)"),
        "roofline": s["roofline"],
        **({"cold": s["cold"]} if "cold" in s else {}),
        **({"warmup_run": s["warmup_run"]} if "warmup_run" in s else {}),
        "device": {"name": props.name, "cus": props.multi_processor_count},
    }
    if "cpu_baseline" in s:
        line["cpu_baseline"] = s["cpu_baseline"]
    if not args.no_cpu_baseline and head in ("prefill", "prefill_nc", "decode_fp8", "decode_bf16"):
        log("cpu baseline ...")
        line["cpu_baseline"] = (cpu_prefill if head.startswith("prefill") else cpu_decode)(r, args.cpu_seconds)
    del r
    torch.cuda.empty_cache()

    if args.workload == "all":
        r = WORKLOADS["decode_fp8"](args.steps, args.warmup)
        log(f"decode_fp8: {r['ms']:.4f} ms/step, {r['value']:.1f} GB/s")
        sec = summary("decode_fp8", r, read_ceiling(args.steps, args.warmup))
        sec["metric"] = "FP8 paged GQA decode HBM GB/s (C4)"
        if not args.no_cpu_baseline:
            sec["cpu_baseline"] = cpu_decode(r, args.cpu_seconds)
        line["fp8_decode"] = sec
        del r
        torch.cuda.empty_cache()
        extra = {}
        for name in ("prefill_nc", "decode_bf16", "mxfp8", "backward", "c1"):
            r = WORKLOADS[name](args.steps, args.warmup)
            log(f"{name}: {r['ms']:.4f} ms/step, {r['value']:.1f} {r['unit']}")
            extra[name] = summary(name, r, read_ceiling(args.steps, args.warmup)
                                  if name.startswith("decode") else None)
            del r
            torch.cuda.empty_cache()
        line["extra"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
