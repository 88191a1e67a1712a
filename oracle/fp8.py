"""FP8 e4m3 (OCP "fn" variant), e8m0 and MX block-scale codecs in numpy.

Test infrastructure only (see ``oracle/__init__.py``).

Reference anchors
-----------------
* e4m3 layout: sign, 4 exponent bits (bias 7), 3 mantissa bits; subnormals
  m * 2^-9; 0x7F / 0xFF are NaN; no infinities. The reference's host emulation
  states the same decode (cuda_compat.h:482-494) but maps NaN to 0 — that quirk
  is not restated here.
* Quantisation recipe: tests/test_kernels_misc.py:52-55 — scale = amax / 448
  clamped at 1e-8, codes = (x / scale).to(torch.float8_e4m3fn), and the oracle
  compares against the *dequantised* values (:57-59). The benchmark config
  moves the scale to one fp32 per (page, kv head), the ``[num_blocks, H]`` form
  the binding accepts (fused_softmax_binding.cpp:640,671).
* MX: the reference only declares the MXFP8 entry point (kernels_api.h:103-108)
  and describes "32-element blocks with a shared e8m0 scale" (README.md:29-31).
  The block-scale rule below is the OCP Microscaling Formats v1.0 definition:
  X = 2^(floor(log2(amax)) - emax_elem), emax_elem = 8 for e4m3, elements
  x / X rounded to nearest-even e4m3 and saturated to +-448.
"""
import numpy as np

E4M3_MAX = 448.0
E4M3_EMAX = 8
MX_BLOCK = 32


def _e4m3_table():
    tab = np.zeros(256, dtype=np.float32)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if e == 0xF and m == 0x7:
            tab[c] = np.nan
        elif e == 0:
            tab[c] = s * m * 2.0 ** -9
        else:
            tab[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return tab


_E4M3 = _e4m3_table()


def e4m3_decode(codes):
    """uint8 e4m3 codes -> float32 values."""
    return _E4M3[np.asarray(codes, dtype=np.uint8)]


def _rne(x):
    return np.round(x)  # numpy rounds half to even


def e4m3_encode(x, saturate=False):
    """float -> uint8 e4m3 codes, round-to-nearest-even.

    ``saturate=False`` follows torch's ``.to(float8_e4m3fn)`` (values whose
    rounding passes 448 become NaN = 0x7F|sign); ``saturate=True`` clamps to
    +-448 first (the MX conversion rule).
    """
    x = np.asarray(x, dtype=np.float64)
    sign = np.signbit(x).astype(np.uint8) << 7
    a = np.abs(x)
    nan = np.isnan(a)
    if saturate:
        a = np.minimum(a, E4M3_MAX)
    inf = np.isinf(a)
    a = np.where(nan | inf, 0.0, a)
    codes = np.zeros(a.shape, dtype=np.int64)
    sub = a < 2.0 ** -6
    # subnormal range (and zero): code = RNE(a / 2^-9); 8 lands on the min normal
    codes = np.where(sub, _rne(a / 2.0 ** -9), codes)
    mant, exp = np.frexp(np.where(sub, 1.0, a))  # a = mant * 2^exp, mant in [0.5, 1)
    e = exp - 1                                   # a = (2*mant) * 2^e, 2*mant in [1, 2)
    m = _rne((2.0 * mant - 1.0) * 8.0)
    carry = m >= 8
    e = np.where(carry, e + 1, e)
    m = np.where(carry, 0, m)
    biased = e + 7
    normal_code = (biased << 3) | m.astype(np.int64)
    overflow = (biased > 15) | ((biased == 15) & (m == 7))
    codes = np.where(sub, codes, normal_code)
    codes = np.where(~sub & overflow, 0x7F, codes)
    codes = np.where(nan | inf, 0x7F, codes)
    return (codes.astype(np.uint8) | sign).astype(np.uint8)


def e8m0_decode(b):
    """uint8 e8m0 (biased exponent, bias 127, 0xFF = NaN) -> float32 2^(b-127)."""
    b = np.asarray(b, dtype=np.uint8).astype(np.int32)
    out = np.ldexp(np.float32(1.0), np.minimum(b, 254) - 127).astype(np.float32)
    return np.where(b == 255, np.float32(np.nan), out).astype(np.float32)


def mx_quantize(x, block=MX_BLOCK):
    """OCP MX v1.0 e4m3 quantisation along the last axis.

    Returns (codes uint8 [..., D], scale_bytes uint8 [..., D // block]).
    An all-zero block gets scale byte 0 (X = 2^-127) and zero codes.
    """
    x = np.asarray(x, dtype=np.float32)
    d = x.shape[-1]
    if d % block:
        raise ValueError(f"last dim {d} not a multiple of the MX block {block}")
    xb = x.reshape(x.shape[:-1] + (d // block, block)).astype(np.float64)
    amax = np.abs(xb).max(axis=-1)
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(amax > 0, amax, 1.0))) - E4M3_EMAX
    e = np.clip(e, -127, 127)
    e = np.where(amax > 0, e, -127).astype(np.int64)
    xs = xb / np.ldexp(1.0, e)[..., None]
    codes = e4m3_encode(xs, saturate=True).reshape(x.shape)
    return codes, (e + 127).astype(np.uint8)


def mx_dequantize(codes, scale_bytes, block=MX_BLOCK):
    """codes [..., D] * 2^(scale-127) per block -> float32 [..., D]."""
    codes = np.asarray(codes, dtype=np.uint8)
    d = codes.shape[-1]
    vals = e4m3_decode(codes).reshape(codes.shape[:-1] + (d // block, block))
    return (vals * e8m0_decode(scale_bytes)[..., None]).reshape(codes.shape).astype(np.float32)


def quantize_per_page_fp8(pages):
    """Per-(page, kv-head) e4m3 quantisation of a paged cache.

    pages: float32 [P, Hkv, D, page] -> (codes uint8 same shape, scale f32 [P, Hkv])
    with scale = max(amax / 448, 1e-8) as in tests/test_kernels_misc.py:52-53.
    """
    pages = np.asarray(pages, dtype=np.float32)
    amax = np.abs(pages).max(axis=(2, 3))
    scale = np.maximum(amax / np.float32(E4M3_MAX), np.float32(1e-8)).astype(np.float32)
    codes = e4m3_encode(pages / scale[:, :, None, None])
    return codes, scale
