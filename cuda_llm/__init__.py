"""Drop-in ``cuda_llm`` namespace (README.md:64-81 of the reference).

``import cuda_llm as cllm`` exposes the same functions as the reference's
extension module (``fused_online_softmax_cuda``): flash_attention /
flash_attention_forward / flash_attention_v3_hopper, fused_gqa_forward,
flash_decode / async_flash_decode, paged_attention(_forward),
fp8_paged_attention(_forward) and fused_microscaled_attention, implemented by
the gfx950 kernels of ``cuda_amd``.
"""
from cuda_amd.api import *  # noqa: F401,F403
from cuda_amd.api import __all__  # noqa: F401
