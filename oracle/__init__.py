"""CPU oracle for the attention forward hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the fp32 math references that the reference
repository uses as its specification (``tests/_utils.py:1-5``: "references
compute in float32 and are the *specification* the CUDA kernels must match"),
plus the data formats on the path (paged KV layout, FP8 e4m3, MX e8m0 block
scales) and CPU restatements of the blocked algorithms the HIP kernels use
(tiled online softmax, split-K with a log-sum-exp merge).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it, and only as the checker or as the timed CPU
baseline. The product path (``cuda_amd``) never imports it and has no CPU
fallback.

Pinning (what checks each function; see ``tests/test_oracle.py``):
  attention / decode / paged_decode  fp64 brute-force loops on tiny shapes,
                                     torch SDPA (CPU, fp32), closed-form
                                     invariants, committed golden fixtures
  e4m3_decode / e4m3_encode          all 256 codes and a dense value sweep
                                     against torch.float8_e4m3fn
  e8m0_decode                        all 256 codes against torch.float8_e8m0fnu
  mx_quantize                        OCP MX v1.0 closed form (scale exponent,
                                     saturation) and round-trip bounds
  attention_tiled / split_merge      equality with ``attention`` (restatements
                                     of the kernels' blocking)
  paged_append                       make_paged_cache of whole sequences,
                                     token-by-token == all at once,
                                     quantize_per_page_fp8 of the built cache,
                                     the per-head e4m3(x / s) recipe
  apply_rope / rope_attention        the complex-number form of the rotation,
                                     norm preservation, position 0 = identity,
                                     torch SDPA of the rotated tensors
  attention_backward                 torch autograd (CPU, fp64) of SDPA,
                                     central finite differences of
                                     ``attention`` (fp64), the one-key closed
                                     form (dq = dk = 0, dv = dout)
No function is left "parity unpinned" except the MXFP8 *semantics* as a whole:
the reference declares ``dispatch_fused_microscaled_attention``
(kernels_api.h:103-108) but ships no kernel, binding or test for it, so the
oracle follows the OCP MX v1.0 definition instead of a reference vector.
"""
from .attention import (apply_rope, attention, attention_backward, attention_lse,
                        attention_tiled, decode, default_scale, rope_attention, split_merge)
from .fp8 import (E4M3_MAX, e4m3_decode, e4m3_encode, e8m0_decode,
                  mx_dequantize, mx_quantize, quantize_per_page_fp8)
from .paged import gather_paged, make_paged_cache, paged_append, paged_decode

__all__ = [
    "apply_rope", "rope_attention", "attention", "attention_backward", "attention_lse", "attention_tiled", "decode", "default_scale",
    "split_merge", "E4M3_MAX", "e4m3_decode", "e4m3_encode", "e8m0_decode",
    "mx_dequantize", "mx_quantize", "quantize_per_page_fp8", "gather_paged",
    "make_paged_cache", "paged_append", "paged_decode",
]
