#!/usr/bin/env python3
"""Benchmark of the attention forward hot path on one MI355X.

Headline line (BASELINE.json metric, config C2): bf16 causal prefill,
q/k/v ~ N(0,1) [4, 32, 4096, 128], fp32 accumulate, bf16 out, inputs resident
in HBM. A step is one ``cuda_llm.flash_attention`` call; FLOPs per step follow
the reference's convention 2*B*H*S^2*D for causal (benchmark_pytorch.py:115-117).
The same JSON line carries, under "fp8_decode", the second half of the
metric: FP8 paged GQA decode at config C4 (N=256, Hq=32/Hkv=8, D=128,
L ~ U[2048, 32768], e4m3 cache with per-(page, kv-head) scales), whose
algorithmic bytes are the K/V bytes of the context tokens plus scales, q, out
and block-table entries.

Timing: W untimed warm-up steps, then K steps between HIP events recorded on
the stream the kernels run on (torch's current stream), bracketed by
device synchronisation. ``cpu_baseline`` times the numpy oracle on a bounded
sample of the same workload on this host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-secondary]
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16/fp16 MFMA (published)
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E (published)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_steps(fn, steps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per step


def _traffic(key):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, copy-kernel calibrated), committed in profiles/traffic.json."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)[key]
        return float(t["fetch_bytes"]) + float(t["write_bytes"])
    except (OSError, KeyError, ValueError, TypeError):
        return None


def blas_threads():
    try:
        from threadpoolctl import threadpool_info
        n = [i.get("num_threads", 0) for i in threadpool_info() if i.get("user_api") == "blas"]
        return max(n) if n else os.cpu_count()
    except Exception:
        return os.cpu_count()


# ---------------------------------------------------------------------------
# C2 prefill
# ---------------------------------------------------------------------------
def bench_prefill(steps, warmup, causal=True, B=4, H=32, S=4096, D=128):
    import torch
    import cuda_llm
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    q, k, v = (torch.randn(B, H, S, D, device="cuda", generator=g).to(torch.bfloat16) for _ in range(3))
    fn = lambda: cuda_llm.flash_attention(q, k, v, is_causal=causal)
    ms = time_steps(fn, steps, warmup)
    flops = (2.0 if causal else 4.0) * B * H * S * S * D
    return dict(ms=ms, flops=flops, tflops=flops / (ms * 1e-3) / 1e12, q=q, k=k, v=v)


def cpu_baseline_prefill(q, k, v, causal, seconds):
    """Oracle (numpy fp32) on as many (b, h) heads of the same inputs as fit in
    ~``seconds``; heads are independent, so the rate scales exactly."""
    import oracle
    B, H, S, D = q.shape
    pairs = [(b, h) for b in range(B) for h in range(H)]
    done = 0
    el = 0.0  # oracle time only; device->host copies are excluded
    for (b, h) in pairs:
        qq = q[b:b + 1, h:h + 1].float().cpu().numpy()
        kk = k[b:b + 1, h:h + 1].float().cpu().numpy()
        vv = v[b:b + 1, h:h + 1].float().cpu().numpy()
        t1 = time.perf_counter()
        oracle.attention(qq, kk, vv, is_causal=causal)
        el += time.perf_counter() - t1
        done += 1
        if el >= seconds:
            break
    flops = (2.0 if causal else 4.0) * S * S * D * done
    return dict(value=flops / el / 1e12, unit="TFLOP/s", cores=blas_threads(), kind="port",
                sample=f"{done} of {B * H} (b,h) heads of the same C2 inputs, numpy fp32 oracle "
                       f"(oracle/attention.py), {el:.1f} s")


# ---------------------------------------------------------------------------
# C4 FP8 paged decode
# ---------------------------------------------------------------------------
def make_c4(seed=0, N=256, Hq=32, Hkv=8, D=128, lo=2048, hi=32768):
    import torch
    gc = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (N,), generator=gc)
    pages = (lens + 15) // 16
    P = int(pages.sum())
    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    perm = torch.randperm(P, device=dev, generator=g).to(torch.int32)
    max_blocks = int(pages.max())
    tables = torch.zeros(N, max_blocks, dtype=torch.int32, device=dev)
    starts = torch.cumsum(pages, 0) - pages
    for i in range(N):
        tables[i, :int(pages[i])] = perm[int(starts[i]):int(starts[i]) + int(pages[i])]
    kc = torch.empty(P, Hkv, D, 16, dtype=torch.uint8, device=dev)
    vc = torch.empty_like(kc)
    ks = torch.empty(P, Hkv, dtype=torch.float32, device=dev)
    vs = torch.empty_like(ks)
    chunk = 32768
    for c0 in range(0, P, chunk):
        c1 = min(P, c0 + chunk)
        for cache, sc in ((kc, ks), (vc, vs)):
            x = torch.randn(c1 - c0, Hkv, D, 16, device=dev, generator=g)
            s = (x.abs().amax(dim=(2, 3)) / 448.0).clamp_min(1e-8)
            cache[c0:c1] = (x / s[:, :, None, None]).to(torch.float8_e4m3fn).view(torch.uint8)
            sc[c0:c1] = s
    q = torch.randn(N, Hq, D, device=dev, generator=g).to(torch.bfloat16)
    lens_d = lens.to(torch.int32).to(dev)
    total_tokens = int(lens.sum())
    alg_bytes = (total_tokens * Hkv * D * 2          # K + V e4m3 codes of the context tokens
                 + int(pages.sum()) * Hkv * 4 * 2    # k/v scales of the pages read
                 + 2 * N * Hq * D * 2                # q in, out
                 + int(pages.sum()) * 4 + N * 4)     # block-table entries, context lengths
    return dict(query=q, kc=kc, vc=vc, ks=ks, vs=vs, tables=tables, lens=lens_d,
                lens_host=lens.tolist(), alg_bytes=alg_bytes, P=P)


def bench_fp8_decode(steps, warmup):
    import torch
    import cuda_llm
    c = make_c4()
    fn = lambda: cuda_llm.fp8_paged_attention_forward(c["query"], c["kc"], c["vc"], c["ks"], c["vs"],
                                                      c["tables"], c["lens"])
    ms = time_steps(fn, steps, warmup)
    gbs = c["alg_bytes"] / (ms * 1e-3) / 1e9
    return dict(ms=ms, gbs=gbs, case=c)


def cpu_baseline_decode(c, seconds):
    import numpy as np
    import oracle
    done_tokens = 0
    done = 0
    t0 = time.perf_counter()
    el = 0.0
    for i in range(len(c["lens_host"])):
        L = c["lens_host"][i]
        nb = (L + 15) // 16
        ids = c["tables"][i, :nb].long()
        kc = c["kc"].index_select(0, ids).cpu().numpy()
        vc = c["vc"].index_select(0, ids).cpu().numpy()
        ks = c["ks"].index_select(0, ids).cpu().numpy()
        vs = c["vs"].index_select(0, ids).cpu().numpy()
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
                kind="port", sample=f"{done} of {len(c['lens_host'])} sequences of the same C4 inputs, "
                                    f"numpy oracle (oracle/paged.py), {el:.1f} s")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-secondary", action="store_true", help="skip the FP8 decode measurement")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    args = ap.parse_args()
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

    log("prefill C2 ...")
    pf = bench_prefill(args.steps, args.warmup)
    log(f"prefill: {pf['ms']:.3f} ms/step, {pf['tflops']:.1f} TFLOP/s")
    line = {
        "metric": "prefill TFLOP/s (bf16 causal, B=4 H=32 S=4096 D=128)",
        "value": round(pf["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pf["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: q/k/v ~ N(0,1) cast to bf16, seed 0, resident in HBM",
        "config": {"workload": "C2 bf16 causal prefill (flash_attention)", "batch": 4, "heads": 32,
                   "seq_len": 4096, "head_dim": 128, "causal": True, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(pf["tflops"], 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(pf["tflops"] / PEAK_BF16_TFLOPS, 4),
                     "traffic": _traffic("prefill_c2_causal")},
        "device": {"name": props.name, "cus": props.multi_processor_count},
    }
    if not args.no_cpu_baseline:
        log("cpu baseline (prefill) ...")
        line["cpu_baseline"] = cpu_baseline_prefill(pf["q"], pf["k"], pf["v"], True, args.cpu_seconds)
    del pf
    torch.cuda.empty_cache()

    if not args.no_secondary:
        log("fp8 paged decode C4 ...")
        dc = bench_fp8_decode(args.steps, args.warmup)
        log(f"fp8 decode: {dc['ms']:.3f} ms/step, {dc['gbs']:.1f} GB/s")
        sec = {
            "metric": "FP8 paged GQA decode HBM GB/s (C4)",
            "value": round(dc["gbs"], 1), "unit": "GB/s", "ms_per_step": round(dc["ms"], 4),
            "dtype": "e4m3 KV, bf16 q/out, fp32 softmax",
            "config": {"workload": "C4 FP8 paged decode", "num_seqs": 256, "q_heads": 32,
                       "kv_heads": 8, "head_dim": 128, "page": 16, "context": "U[2048, 32768]",
                       "pool_pages": dc["case"]["P"], "alg_bytes_per_step": dc["case"]["alg_bytes"]},
            "roofline": {"bound": "hbm", "achieved": round(dc["gbs"], 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(dc["gbs"] / PEAK_HBM_GBS, 4),
                         "traffic": _traffic("fp8_decode_c4")},
        }
        if not args.no_cpu_baseline:
            log("cpu baseline (decode) ...")
            sec["cpu_baseline"] = cpu_baseline_decode(dc["case"], args.cpu_seconds)
        line["fp8_decode"] = sec
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
