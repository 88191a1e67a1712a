"""The reference's extension module name, importable unchanged.

The reference's tests and benchmark ``import fused_online_softmax_cuda``
(tests/conftest.py:25, setup.py:128, benchmark_pytorch.py) and call the
functions its pybind11 module defines (fused_softmax_binding.cpp:721-809).
This module binds those names to this build's gfx950 entry points, with the
same argument names and defaults. The module's other functions (``forward``:
the standalone online softmax, ``fused_mla_forward``,
``fused_llama_megablock``) belong to subsystems outside the attention forward
path and are not provided: looking them up raises AttributeError, as it does
for a reference build compiled without them (the WITH_* guards of
fused_softmax_binding.cpp).
"""
from cuda_amd.api import (  # noqa: F401
    async_flash_decode,
    flash_attention_backward,
    flash_attention_forward,
    flash_attention_v3_hopper,
    fp8_paged_attention_forward,
    fused_gqa_forward,
    fused_microscaled_attention,
    fused_rope_flash_attention,
    paged_attention_forward,
)

_NOT_BUILT = ("forward", "fused_mla_forward", "fused_llama_megablock")


def __getattr__(name):
    if name in _NOT_BUILT:
        raise AttributeError(
            f"fused_online_softmax_cuda.{name} is outside the attention forward path this "
            "build provides (see cuda_llm for the entry points that are)")
    raise AttributeError(f"module 'fused_online_softmax_cuda' has no attribute {name!r}")
