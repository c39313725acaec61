"""Walsh-Hadamard rotation and fp4 e2m1 block act-quant of the indexer keys (CPU oracle).

Restates ``v4mlx/qat.py``, the key-side transform of the indexer compressor
(``v4mlx/compressor.py:57-59``: Hadamard over all channels, then fp4 over all channels):

* ``hadamard_rotate`` (``v4mlx/qat.py:8-20``): the in-place butterfly over the last dim, stages
  h = 1, 2, 4, ..., n/2; at stage h each group of 2h values (a_j, b_j) = (x[2hg+j], x[2hg+h+j])
  becomes (a_j + b_j, a_j - b_j); every add is one float32 rounding.  Then a float32 multiply by
  float32(n ** -0.5).
* ``fp4_act_quant`` (``v4mlx/qat.py:23-31``): per block of 32, ``amax = max(|x|, 6 * 2**-126)``,
  ``s = 2**ceil(log2(amax / 6))``, ``q = e2m1(clip(x / s, -6, 6)) * s`` with e2m1 round to nearest,
  ties to the even code.  The grid is {0, 0.5, 1, 1.5, 2, 3, 4, 6}.
* ``fp4_quantize``: the stored form of the same quantisation (the form the HIP kernel writes):
  packed e2m1 codes (element 2i in the low nibble of byte i, bit 3 the sign) and one ue8m0 scale
  byte per block (log2(s) + 127); ``fp4_dequantize`` decodes it (the indexer's fp4 keys).

The scale exponent is computed exactly from the float32 bits of ``amax / 6`` (the unbiased
exponent, plus one unless the value is a power of two).  The reference takes a float32 ``log2``
then ``ceil``.  The two disagree only where float32 ``log2`` rounds a value a few ulps above a
power of two down onto the integer.  That happens for a handful of float32 values per binade,
and no test input hits one.

Pinning (``tests/test_oracle_qat.py``):
* the rotation equals ``scipy.linalg.hadamard(n) @ x * n**-0.5`` exactly on small-integer inputs,
  where every sum is exact, and within float32 rounding on random inputs;
* the float32 rounding order equals Sylvester's recursion H_2m x = [H_m x0 + H_m x1; H_m x0 - H_m x1]
  computed bottom-up, on random inputs, bit for bit;
* e2m1 rounding equals a brute-force nearest search over the 15 values with ties to the even code,
  on every midpoint and on random values;
* the scale equals a brute-force search for the smallest power of two s with fl32(amax/6) <= s;
* the decode equals the OCP MX definition (sign, 2-bit exponent, 1-bit mantissa; E8M0 scale,
  0xFF NaN) evaluated exactly in rationals, for every code byte and every scale byte.
``ml_dtypes`` is absent here, so its own float4 cast is parity unpinned beyond agreeing with that
definition.
"""
import numpy as np

FP4_MAX = 6.0
FP4_GRID = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)
AMAX_FLOOR = np.float32(6.0 * 2.0 ** -126)


def rotate_scale(n):
    """float32(n ** -0.5), the multiplier after the butterfly (``v4mlx/qat.py:20``)."""
    return np.float32(n ** -0.5)


def hadamard_rotate(x):
    """x [..., n] (n a power of two) -> float32 [..., n]."""
    a = np.array(x, dtype=np.float32, copy=True)
    n = a.shape[-1]
    assert n > 0 and (n & (n - 1)) == 0, "Hadamard needs a power-of-two last dim"
    lead = a.shape[:-1]
    h = 1
    while h < n:
        v = a.reshape(*lead, n // (2 * h), 2, h)
        lo, hi = v[..., 0, :], v[..., 1, :]
        a = np.stack([lo + hi, lo - hi], axis=-2).reshape(*lead, n)
        h *= 2
    return (a * rotate_scale(n)).astype(np.float32)


def e2m1_code(z):
    """float32 z with |z| <= 6 -> e2m1 code 0..15 (bit 3 sign), round to nearest, ties to even."""
    z = np.asarray(z, dtype=np.float32)
    a = np.abs(z)
    # the code is the number of decision points passed; ties go to the even code, so the points
    # between an even code and the next odd one are strict, the others inclusive
    mag = ((a > 0.25).astype(np.int64) + (a >= 0.75) + (a > 1.25) + (a >= 1.75) + (a > 2.5) + (a >= 3.5)
           + (a > 5.0))
    sign = np.signbit(z).astype(np.int64)
    return (mag | (sign << 3)).astype(np.uint8)


def e2m1_value(code):
    """e2m1 code (0..15) -> float32 (sign bit kept, so code 8 is -0.0)."""
    c = np.asarray(code, dtype=np.int64)
    v = FP4_GRID[c & 7]
    return np.where(c & 8, -v, v).astype(np.float32)


def fp4_scale_exponent(amax):
    """Exact ceil(log2(fl32(max(amax, 6*2^-126) / 6))) as int64, for float32 amax >= 0."""
    a = np.maximum(np.asarray(amax, dtype=np.float32), AMAX_FLOOR)
    v = (a / np.float32(FP4_MAX)).astype(np.float32)
    bits = v.view(np.uint32).astype(np.int64)
    e = ((bits >> 23) & 0xFF) - 127                  # v >= 2^-126: always a normal number
    return np.where((bits & 0x7FFFFF) == 0, e, e + 1)


def _blocks(x, block):
    a = np.asarray(x, dtype=np.float32)
    assert a.shape[-1] % block == 0
    return a.reshape(*a.shape[:-1], a.shape[-1] // block, block)


def fp4_quantize(x, block=32):
    """x [..., n] float32 -> (packed codes uint8 [..., n/2], ue8m0 scales uint8 [..., n/block])."""
    ab = _blocks(x, block)
    amax = np.abs(ab).max(-1, keepdims=True)
    k = fp4_scale_exponent(amax)
    z = np.clip(ab * np.exp2(-k).astype(np.float32), -FP4_MAX, FP4_MAX).astype(np.float32)
    codes = e2m1_code(z).reshape(*ab.shape[:-2], -1).astype(np.uint8)
    packed = (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)
    return packed, (k[..., 0] + 127).astype(np.uint8)


def ue8m0_value(scales):
    """ue8m0 scale bytes -> float32 2^(b - 127); byte 0 is the subnormal 2^-127, byte 255 NaN."""
    b = np.asarray(scales, dtype=np.int64)
    s = np.exp2(np.minimum(b, 254) - 127).astype(np.float32)
    return np.where(b == 255, np.float32(np.nan), s).astype(np.float32)


def fp4_dequantize(packed, scales, block=32):
    """Inverse of the stored form: float32 [..., 2 * packed.shape[-1]], each value the exact
    float32 product e2m1(code) * 2^(scale - 127) (overflow to inf, NaN for scale byte 255)."""
    p = np.asarray(packed, dtype=np.uint8)
    codes = np.stack([p & 15, p >> 4], axis=-1).reshape(*p.shape[:-1], -1)
    v = e2m1_value(codes)
    s = ue8m0_value(scales)
    vb = v.reshape(*v.shape[:-1], v.shape[-1] // block, block) * s[..., None]
    return vb.reshape(v.shape).astype(np.float32)


def fp4_act_quant(x, block=32):
    """The reference's round trip: float32 [..., n] -> float32 [..., n]."""
    packed, scales = fp4_quantize(x, block)
    return fp4_dequantize(packed, scales, block)


def rotate_fp4(x, block=32):
    """The indexer compressor's key transform: fp4_act_quant(hadamard_rotate(x))."""
    return fp4_act_quant(hadamard_rotate(x), block)
