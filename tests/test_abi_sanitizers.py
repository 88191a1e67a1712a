"""CPU tier: the C ABI's host code under AddressSanitizer and
UndefinedBehaviorSanitizer.

abi.cpp (every entry point's argument checks, workspace sizes and error
messages) is compiled with both sanitizers on the host side only (a HIP
build's device code cannot take them), linked with
tests/abi_checks_harness.cpp and resolved against the built library for the
kernel launchers. The harness makes only calls that are rejected, or have
nothing to do, before the GPU is touched, so it runs on a machine without
one; a sanitizer report or a failed expectation fails the test.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROCM = "/opt/rocm"
HIPCC = os.path.join(ROCM, "bin", "hipcc")
CLANG = os.path.join(ROCM, "llvm", "bin", "clang++")
LIB_DIR = os.path.join(ROOT, "cuda_amd")


def _run(cmd, **kw):
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600, **kw)
    assert r.returncode == 0, f"{' '.join(cmd[:3])} ...\n{r.stdout[-3000:]}\n{r.stderr[-3000:]}"
    return r


def test_abi_checks_under_sanitizers(tmp_path):
    if not os.path.exists(os.path.join(LIB_DIR, "libcuda_llm_amd.so")):
        pytest.skip("library not built (python -m cuda_amd.build)")
    if not (os.path.exists(HIPCC) and os.path.exists(CLANG)):
        pytest.skip("ROCm compilers absent")
    abi_o, harness_o, exe = (str(tmp_path / n) for n in ("abi.o", "harness.o", "abi_checks"))
    _run([HIPCC, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fno-omit-frame-pointer",
          "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
          "-Xarch_host", "-fno-sanitize-recover=all",
          "-x", "hip", "-c", os.path.join(LIB_DIR, "csrc", "abi.cpp"), "-o", abi_o])
    _run([CLANG, "-O1", "-g", "-std=c++17", "-fno-omit-frame-pointer",
          "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
          "-c", os.path.join(ROOT, "tests", "abi_checks_harness.cpp"), "-o", harness_o])
    _run([CLANG, "-fsanitize=address,undefined", abi_o, harness_o, "-o", exe,
          f"-L{LIB_DIR}", "-lcuda_llm_amd", f"-Wl,-rpath,{LIB_DIR}",
          f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib"])
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = _run([exe], env=env)
    assert "abi checks: all passed" in r.stdout, r.stdout + r.stderr
