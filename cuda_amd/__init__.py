"""MI355X (gfx950) attention forward hot path of ``cuda_llm``.

``cuda_amd.api`` holds the reference's Python API (the pybind11 module
functions of fused_softmax_binding.cpp and the README's ``cuda_llm`` names);
``cuda_amd._lib`` binds the C ABI of ``include/cuda_llm_abi.h``; the HIP
kernels live in ``cuda_amd/csrc`` and are built by ``cuda_amd.build``.
"""
from .api import *  # noqa: F401,F403
from .api import __all__  # noqa: F401
