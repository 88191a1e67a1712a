"""ctypes binding of the C ABI (``include/cuda_llm_abi.h``).

Loads the in-tree ``libcuda_llm_amd.so`` built by ``cuda_amd.build``. There is
no fallback: if the library is missing or fails to load, every entry point
raises, so a GPU run can never silently use a CPU path.
"""
import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libcuda_llm_amd.so")

CA_OK, CA_INVALID_ARGUMENT, CA_UNSUPPORTED, CA_LAUNCH_FAILED = 0, 1, 2, 3
CA_F32, CA_F16, CA_BF16 = 0, 1, 2
CA_SCALE_E8M0, CA_SCALE_F32 = 0, 1

#: exported symbol -> (restype, argtypes); the single source of truth for the
#: ABI surface, checked against include/cuda_llm_abi.h by the CPU tests.
_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_Z = ctypes.c_size_t
SIGNATURES = {
    "ca_flash_attention_fwd": (_I, [_I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _P]),
    "ca_flash_attention_fwd_lse": (_I, [_I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _P]),
    "ca_flash_attention_bwd": (_I, [_I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F,
                                    _I, _P, _Z, _P]),
    "ca_flash_attention_bwd_workspace_bytes": (_Z, [_I, _I, _I]),
    "ca_fused_rope_flash_attention": (_I, [_I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I,
                                           _P, _Z, _P]),
    "ca_rope_workspace_bytes": (_Z, [_I, _I, _I, _I, _I, _I]),
    "ca_stream_read": (_I, [_P, _Z, _P, _P]),
    "ca_paged_kv_append": (_I, [_I, _I, _P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I,
                                _I, _P]),
    "ca_flash_decode": (_I, [_I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _Z, _P]),
    "ca_paged_attention": (_I, [_I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P, _Z, _P]),
    "ca_fp8_paged_attention": (_I, [_I, _P, _P, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P, _Z, _P]),
    "ca_fp8_paged_attention_noalloc": (_I, [_I, _P, _P, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P]),
    "ca_fused_microscaled_attention": (_I, [_I, _P, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _F,
                                            _I, _P, _Z, _P]),
    "ca_mx_workspace_bytes": (_Z, [_I, _I, _I, _I, _I]),
    "ca_decode_workspace_bytes": (_Z, [_I, _I, _I, _I]),
    "ca_check_block_tables": (_I, [_P, _P, _I, _I, _I, _I, _P]),
    "ca_check_mx_scales": (_I, [_P, _P, _P, _I, _I, _I, _I, _P]),
    "ca_last_error": (ctypes.c_char_p, []),
    "ca_version": (ctypes.c_char_p, []),
}

_lib = None
_lock = threading.Lock()


class LibraryNotBuilt(RuntimeError):
    pass


def load():
    """Load (once) and return the ctypes library handle."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise LibraryNotBuilt(
                    f"{LIB_PATH} is missing: build it with `python -m cuda_amd.build` "
                    "(there is no CPU fallback)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def call(name, *args):
    """Call an ABI entry point; raise RuntimeError with the library's message
    on a non-OK status (the reference raises via TORCH_CHECK)."""
    lib = load()
    st = getattr(lib, name)(*args)
    if st != CA_OK:
        msg = lib.ca_last_error().decode(errors="replace")
        kind = {CA_INVALID_ARGUMENT: "invalid argument", CA_UNSUPPORTED: "unsupported",
                CA_LAUNCH_FAILED: "launch failed"}.get(st, f"status {st}")
        raise RuntimeError(f"{msg} [{kind}]")
    return st
