"""The Hadamard rotation and fp4 e2m1 quantisation of the oracle, pinned without the reference.

Each check is independent of the oracle's own formula: scipy's Hadamard matrix, Sylvester's
recursion for the rounding order, a brute-force nearest search for e2m1, a brute-force power-of-two
search for the scale.  A planted mistake (a descending stage order, ties away from zero, a scale one
binade off) fails one of them."""
from fractions import Fraction

import numpy as np
import pytest
import scipy.linalg

from oracle import qat

NS = [32, 64, 128, 256, 512, 1024]


def _sylvester(x):
    """H_n x by Sylvester's recursion, in float32: H_2m [x0; x1] = [H_m x0 + H_m x1; H_m x0 - H_m x1]."""
    n = x.shape[-1]
    if n == 1:
        return x.astype(np.float32)
    a = _sylvester(x[..., : n // 2])
    b = _sylvester(x[..., n // 2:])
    return np.concatenate([a + b, a - b], axis=-1).astype(np.float32)


@pytest.mark.parametrize("n", NS)
def test_hadamard_matches_scipy_exactly_on_integers(n):
    rng = np.random.default_rng(n)
    x = rng.integers(-8, 9, size=(5, n)).astype(np.float32)   # every partial sum exact in float32
    got = qat.hadamard_rotate(x)
    ref = (x.astype(np.float64) @ scipy.linalg.hadamard(n).T.astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(got, (ref * qat.rotate_scale(n)).astype(np.float32))


@pytest.mark.parametrize("n", NS)
def test_hadamard_random_close_to_scipy_and_orthonormal(n):
    rng = np.random.default_rng(n + 1)
    x = rng.standard_normal((7, n)).astype(np.float32)
    got = qat.hadamard_rotate(x).astype(np.float64)
    ref = x.astype(np.float64) @ scipy.linalg.hadamard(n).T * n ** -0.5
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-5 * np.sqrt(n))
    # orthonormal: norms kept, applying it twice gives x back
    np.testing.assert_allclose(np.linalg.norm(got, axis=1), np.linalg.norm(x, axis=1), rtol=1e-5)
    np.testing.assert_allclose(qat.hadamard_rotate(qat.hadamard_rotate(x)), x, atol=1e-5)


@pytest.mark.parametrize("n", NS)
def test_hadamard_rounding_order_is_sylvester_bottom_up(n):
    rng = np.random.default_rng(n + 2)
    x = (rng.standard_normal((9, n)) * np.exp2(rng.integers(-20, 20, (9, n)))).astype(np.float32)
    got = qat.hadamard_rotate(x)
    ref = (_sylvester(x) * qat.rotate_scale(n)).astype(np.float32)
    np.testing.assert_array_equal(got, ref)
    # the opposite stage order (largest stride first) rounds differently on these inputs
    a = x.copy()
    h = n // 2
    while h >= 1:
        v = a.reshape(9, n // (2 * h), 2, h)
        a = np.stack([v[:, :, 0] + v[:, :, 1], v[:, :, 0] - v[:, :, 1]], axis=2).reshape(9, n)
        h //= 2
    assert not np.array_equal((a * qat.rotate_scale(n)).astype(np.float32), got)


def test_rotate_scale_values():
    for n in NS:
        k = int(np.log2(n))
        want = np.float32(2.0 ** -(k // 2)) * (np.float32(np.sqrt(0.5)) if k % 2 else np.float32(1))
        assert qat.rotate_scale(n) == np.float32(want)


def _e2m1_brute(z):
    vals = np.array([qat.e2m1_value(c) for c in range(16)], dtype=np.float64)
    out = np.empty(z.shape, dtype=np.uint8)
    for i, v in enumerate(z.ravel()):
        d = np.abs(vals - float(v))
        # among codes of the value's own sign (zero keeps the sign of the input)
        cand = [c for c in range(16) if (c >> 3) == int(np.signbit(v))]
        best = min(d[c] for c in cand)
        ties = [c for c in cand if d[c] == best]
        even = [c for c in ties if (c & 1) == 0]
        out.ravel()[i] = even[0] if even else ties[0]
    return out


def test_e2m1_rounding_brute_force():
    grid = qat.FP4_GRID.astype(np.float64)
    mids = (grid[1:] + grid[:-1]) / 2
    pts = np.concatenate([grid, mids, np.nextafter(mids.astype(np.float32), 0), np.nextafter(mids.astype(np.float32), 7)])
    pts = np.concatenate([pts, -pts]).astype(np.float32)
    rng = np.random.default_rng(3)
    pts = np.concatenate([pts, rng.uniform(-6, 6, 4000).astype(np.float32)])
    np.testing.assert_array_equal(qat.e2m1_code(pts), _e2m1_brute(pts))
    # ties at the midpoints go to the even code: 0.25->0, 0.75->1, 1.25->1, 1.75->2, 2.5->2, 3.5->4, 5->4
    np.testing.assert_array_equal(qat.e2m1_value(qat.e2m1_code(mids.astype(np.float32))),
                                  np.array([0, 1, 1, 2, 2, 4, 4], dtype=np.float32))


def test_scale_exponent_brute_force():
    rng = np.random.default_rng(4)
    amax = np.concatenate([
        (rng.uniform(0.5, 1, 3000) * np.exp2(rng.integers(-140, 120, 3000))).astype(np.float32),
        np.float32(6.0) * np.exp2(np.arange(-126, 126)).astype(np.float32),     # exact powers
        [0.0, 1e-45, np.float32(3.4e38)],
    ]).astype(np.float32)
    k = qat.fp4_scale_exponent(amax)
    v = (np.maximum(amax, qat.AMAX_FLOOR) / np.float32(6.0)).astype(np.float64)
    for vi, ki in zip(v, k):
        kb = -200
        while 2.0 ** kb < vi:
            kb += 1
        assert ki == kb, (vi, ki, kb)


def test_fp4_act_quant_properties():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((64, 256)) * np.exp2(rng.integers(-30, 30, (64, 1)))).astype(np.float32)
    x[0] = 0.0
    x[1, :32] = 6.0 * 2.0 ** 5         # a block at an exact power of two times 6
    x[2, 40] = -1e-30
    q = qat.fp4_act_quant(x)
    packed, scales = qat.fp4_quantize(x)
    s = np.exp2(scales.astype(np.int64) - 127)
    # every block: max |x|/s in (3, 6], each value within half a grid step of its quantisation
    ab = np.abs(x).reshape(64, 8, 32).max(-1)
    live = ab > 0
    assert np.all((ab / s)[live] <= 6.0) and np.all((ab / s)[live] > 3.0)
    np.testing.assert_array_equal(q[0], 0.0)
    np.testing.assert_array_equal(q[1, :32], 6.0 * 2.0 ** 5)
    err = np.abs(q - x) / np.repeat(s, 32, axis=1)
    assert np.all(err <= 1.0 + 1e-6)      # grid step is at most 2 (between 4 and 6)
    # idempotent, and the stored form decodes to the round trip
    np.testing.assert_array_equal(qat.fp4_act_quant(q), q)
    np.testing.assert_array_equal(qat.fp4_dequantize(packed, scales), q)
    assert packed.shape == (64, 128) and scales.shape == (64, 8)


def test_rotate_fp4_composition():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((4, 128)).astype(np.float32)
    np.testing.assert_array_equal(qat.rotate_fp4(x), qat.fp4_act_quant(qat.hadamard_rotate(x)))


def _e2m1_ocp(c):
    """OCP MX FP4 (E2M1): sign bit 3, exponent bits 2..1 (bias 1), mantissa bit 0; exponent 0 is
    subnormal (mantissa / 2)."""
    sign = -1 if c & 8 else 1
    e, m = (c >> 1) & 3, c & 1
    mag = Fraction(m, 2) if e == 0 else Fraction(2) ** (e - 1) * (1 + Fraction(m, 2))
    return sign, mag


def test_fp4_dequantize_matches_ocp_definition():
    """Every packed byte (two codes) under every E8M0 scale byte, against exact rationals rounded
    once to float32 (the product of a grid value and a power of two is exact unless it overflows)."""
    packed = np.arange(256, dtype=np.uint8)[:, None].repeat(256, 1).reshape(256, 256, 1)
    scales = np.arange(256, dtype=np.uint8)[None, :, None].repeat(256, 0)
    got = qat.fp4_dequantize(packed.reshape(-1, 1).repeat(16, 1), scales.reshape(-1, 1), block=32)
    got = got.reshape(256, 256, 32)
    fmax = Fraction(np.finfo(np.float32).max.item())
    for byte in range(256):
        for half, c in enumerate((byte & 15, byte >> 4)):
            sign, mag = _e2m1_ocp(c)
            for sb in range(256):
                v = got[byte, sb, half]
                if sb == 255:
                    assert np.isnan(v), (byte, sb)
                    continue
                exact = mag * Fraction(2) ** (sb - 127)
                if exact > fmax:
                    assert np.isinf(v) and np.sign(v) == sign, (byte, sb, v)
                else:
                    assert Fraction(float(abs(v))) == exact and (np.signbit(v) == (sign < 0)), (byte, sb, v)
