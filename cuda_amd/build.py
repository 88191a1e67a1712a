"""Build the gfx950 shared library ``cuda_amd/libcuda_llm_amd.so`` with hipcc.

Usage: ``python -m cuda_amd.build`` (or ``__graft_entry__.build()``).
Each HIP source is compiled to an object in ``cuda_amd/_build/`` (in
parallel), then linked into the in-tree shared library that
``cuda_amd._lib`` loads. Nothing is hipified: the sources are written for
gfx950 directly.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libcuda_llm_amd.so")
SOURCES = ["prefill.hip", "prefill_w64.hip", "prefill_w64_mx.hip", "decode.hip", "mxfp8.hip", "f32.hip", "backward.hip", "backward_f32.hip",
           "kv_append.hip", "rope.hip", "stream_read.hip", "abi.cpp"]
ARCH = os.environ.get("CA_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # gfx950: keep hipcc from emitting packed-fp32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]
# Per-source additions. prefill: the softmax row max runs on v_max/v_max3;
# with the IEEE mode bit on, every fmaxf operand that does not come from an
# arithmetic instruction (MFMA results do not count) is first quieted with an
# extra v_max. The kernels there have no NaN-dependent logic.
# f32: MFMA accumulators in ordinary VGPRs. The fp32 split-walk kernel's VALU
# reads its S and O accumulators every tile; allocated in AGPRs they cost a
# v_accvgpr_read/write per element and tile (measured: ~130-190 per tile at
# D = 64), which a wave pays in series with its MFMAs. decode: the same for
# the paged walks' O accumulators (rescales and the output pass; C4 5918 ->
# 6601 GB/s with one wave per SIMD).
# backward: the instruction scheduler's max-ILP strategy (same registers, no
# scratch, bitwise-equal gradients): C2 backward 716 -> 727 and 735 -> 748
# TFLOP/s (two A/B runs); it made the 32-row forward at head dim 64 2-3 %
# slower, so it stays on the backward only.
EXTRA = {"prefill.hip": ["-mno-amdgpu-ieee", "-fno-honor-nans"],
         "f32.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
         "decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
         "backward.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]}


# Generated sources: the 64-row prefill's kernel body (hand-scheduled
# assembly, checked for hazards by its generator) is written into the build
# directory before the compile.
GENERATED = {"prefill_w64.hip": ("gen_prefill_w64.py", "prefill_w64_body.inc", ()),
             "prefill_w64_mx.hip": ("gen_prefill_w64.py", "prefill_w64_mx_body.inc", ("--mx",))}


def _generate(src):
    gen, out, flags = GENERATED[src]
    r = subprocess.run([sys.executable, os.path.join(CSRC, gen), *flags, os.path.join(BUILD, out)],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{gen} failed:\n{r.stderr}")


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    if src in GENERATED:
        _generate(src)
    cmd = [HIPCC, *COMMON, *EXTRA.get(src, []), "-I", BUILD, "-x", "hip", "-c", os.path.join(CSRC, src),
           "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose=True):
    """Compile every HIP source and link the shared library. Returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(4, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
