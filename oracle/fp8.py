"""fp8 e4m3fn (OCP, max 448) rounding and the pow2-scale block act-quant (CPU oracle).

Restates:

* the e4m3fn cast the reference takes from ``ml_dtypes.float8_e4m3fn`` (``v4mlx/compressor.py:19``,
  ``oracle/decode_engine.py:54``) and re-derives by hand in ``oracle/step12_glue.py:57-60``:
  round to nearest, ties to even, 3 mantissa bits, subnormal quantum 2**-9;
* ``act_quant_sim`` (``v4mlx/compressor.py:11-20``): per block of 64, ``amax = max(|x|, 1e-4)``,
  ``s = 2**ceil(log2(amax/448))``, ``q = e4m3(clip(x/s, -448, 448)) * s``.

The scale exponent is computed exactly from the float32 bits of ``amax/448`` (ceil(log2(v)) is
the unbiased exponent, plus one unless v is an exact power of two).  The reference takes a float32
``log2`` then ``ceil``; the two agree except where float32 ``log2`` rounds a value just above a
power of two down onto the integer, a measure-zero set that no test input hits.

Pinning: ``e4m3_round`` is checked code-by-code against ``torch.float8_e4m3fn`` (a library
routine) over all 256 codes, every midpoint between neighbouring codes, and random values; the
scale recipe against a brute-force search for the smallest power of two with amax/s <= 448.
``ml_dtypes`` is absent here, so its own rounding is parity unpinned beyond agreeing with torch.
"""
import numpy as np
import torch

E4M3_MAX = 448.0


def e4m3_round(x):
    """Round float32 values to the nearest e4m3fn value (ties to even). |x| must be <= 448.

    Returns float32.  Implemented with integer arithmetic on the float32 bit pattern.
    """
    a = np.asarray(x, dtype=np.float32)
    bits = a.view(np.uint32).astype(np.int64)
    sign = bits & 0x80000000
    mag = bits & 0x7FFFFFFF
    exp = (mag >> 23) - 127                       # unbiased exponent of |x| (normals)
    # quantum (ulp) of the e4m3 grid at this magnitude: 2**(exp-3) for normals (exp >= -6),
    # 2**-9 in the subnormal range.
    qexp = np.maximum(exp, -6) - 3
    absf = np.abs(a.astype(np.float64))
    scaled = absf / np.exp2(qexp.astype(np.float64))          # exact (power-of-two division)
    fl = np.floor(scaled)
    frac = scaled - fl
    up = (frac > 0.5) | ((frac == 0.5) & (np.mod(fl, 2) == 1))
    r = (fl + up) * np.exp2(qexp.astype(np.float64))
    r = np.where(mag == 0, 0.0, r)
    out = r.astype(np.float32)
    return np.where(sign != 0, -out, out).astype(np.float32)


def e4m3_encode(x):
    """float32 (|x| <= 448) -> uint8 e4m3fn code, round to nearest even."""
    r = e4m3_round(x)
    return torch.from_numpy(np.ascontiguousarray(r)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def e4m3_decode(codes):
    """uint8 e4m3fn codes -> float32 (0x7F / 0xFF decode to NaN)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = np.where((e == 0xF) & (m == 0x7), np.nan, val)
    return (s * val).astype(np.float32)


def pow2_scale_exponent(amax):
    """Exact ceil(log2(amax / 448)) for float32 amax > 0, as int64."""
    v = (np.asarray(amax, dtype=np.float32) / np.float32(E4M3_MAX)).astype(np.float32)
    bits = v.view(np.uint32).astype(np.int64)
    e = ((bits >> 23) & 0xFF) - 127
    mant = bits & 0x7FFFFF
    # subnormal v cannot occur: amax >= 1e-4 so v >= 2.2e-7
    return np.where(mant == 0, e, e + 1)


def act_quant_sim(x, block=64):
    """Blockwise fp8 round trip with pow2 scales; returns (dequantized fp32, scales fp32).

    x: [..., n] float32 with n % block == 0.  scales has shape [..., n // block].
    """
    a = np.asarray(x, dtype=np.float32)
    sh = a.shape
    blk = a.reshape(*sh[:-1], sh[-1] // block, block)
    amax = np.maximum(np.abs(blk).max(axis=-1), np.float32(1e-4)).astype(np.float32)
    s = np.exp2(pow2_scale_exponent(amax).astype(np.float64)).astype(np.float32)
    scaled = np.clip(blk / s[..., None], -E4M3_MAX, E4M3_MAX).astype(np.float32)
    q = e4m3_round(scaled) * s[..., None]
    return q.reshape(sh).astype(np.float32), s


def quantize_e4m3_pow2(x, block=64):
    """Blockwise quantisation to (uint8 codes, fp32 pow2 scales) — the stored form of a fp8 cache.

    Decoding ``e4m3_decode(codes) * scale`` gives exactly ``act_quant_sim(x)[0]``.
    """
    a = np.asarray(x, dtype=np.float32)
    sh = a.shape
    blk = a.reshape(*sh[:-1], sh[-1] // block, block)
    amax = np.maximum(np.abs(blk).max(axis=-1), np.float32(1e-4)).astype(np.float32)
    s = np.exp2(pow2_scale_exponent(amax).astype(np.float64)).astype(np.float32)
    scaled = np.clip(blk / s[..., None], -E4M3_MAX, E4M3_MAX).astype(np.float32)
    codes = e4m3_encode(scaled)
    return codes.reshape(sh), s
