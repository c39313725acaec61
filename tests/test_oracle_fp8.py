"""Pins oracle.fp8 against torch.float8_e4m3fn (a library routine) and brute force."""
import numpy as np
import torch

from oracle import fp8


def _all_finite_codes():
    codes = np.arange(256, dtype=np.uint8)
    vals = fp8.e4m3_decode(codes)
    return codes[np.isfinite(vals)], vals[np.isfinite(vals)]


def test_decode_matches_torch_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    ours = fp8.e4m3_decode(codes)
    both_nan = np.isnan(ref) & np.isnan(ours)
    assert np.all(both_nan | (ref == ours))
    assert np.isnan(ours[0x7F]) and np.isnan(ours[0xFF])
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9


def test_round_matches_torch_codes_midpoints_random():
    _, vals = _all_finite_codes()
    pos = np.unique(np.abs(vals))
    mids = ((pos[1:].astype(np.float64) + pos[:-1]) / 2).astype(np.float32)
    rng = np.random.default_rng(0)
    rnd = (rng.standard_normal(20000) * rng.choice([1e-3, 0.1, 1, 30, 200], 20000)).astype(np.float32)
    rnd = np.clip(rnd, -448, 448)
    tiny = np.float32([2.0 ** -10, 2.0 ** -10 * 1.0001, 2.0 ** -11, 3 * 2.0 ** -10, 1e-30, 0.0, -0.0])
    x = np.concatenate([vals, mids, -mids, np.nextafter(mids, 0), np.nextafter(mids, 1), rnd, tiny])
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).float().numpy()
    ours = fp8.e4m3_round(x)
    np.testing.assert_array_equal(ours, ref)


def test_midpoint_ties_go_to_even():
    # 1.0625 is halfway between 1.0 (mantissa 000) and 1.125 (001) -> 1.0 ; 1.1875 -> 1.25
    assert fp8.e4m3_round(np.float32([1.0625]))[0] == 1.0
    assert fp8.e4m3_round(np.float32([1.1875]))[0] == 1.25
    assert fp8.e4m3_round(np.float32([3 * 2.0 ** -10]))[0] == 2.0 ** -8  # subnormal tie -> even


def test_pow2_scale_is_smallest_power_covering_amax():
    rng = np.random.default_rng(1)
    amax = np.concatenate([np.exp2(rng.uniform(-13, 12, 5000)), np.exp2(np.arange(-13, 12)) * 448.0,
                           [1e-4]]).astype(np.float32)
    e = fp8.pow2_scale_exponent(amax)
    for a, ee in zip(amax[:2000], e[:2000]):
        # brute force: smallest integer t with a/448 <= 2^t (in exact float arithmetic)
        t = -40
        while float(a) / 448.0 > 2.0 ** t:
            t += 1
        assert t == ee
    # exact powers of two do not round up
    v = np.float32(448.0 * 2.0 ** 3)
    assert fp8.pow2_scale_exponent(np.array([v]))[0] == 3


def test_act_quant_roundtrip_properties():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((5, 448)) * 0.3).astype(np.float32)
    q, s = fp8.act_quant_sim(x, 64)
    assert s.shape == (5, 7)
    # scale is a power of two and every block's scaled values fit e4m3
    assert np.all(np.frexp(s)[0] == 0.5)
    blk = x.reshape(5, 7, 64)
    assert np.all(np.abs(blk).max(-1) / s <= 448.0)
    # stored form decodes to the same values
    codes, s2 = fp8.quantize_e4m3_pow2(x, 64)
    np.testing.assert_array_equal(s, s2)
    dec = (fp8.e4m3_decode(codes).reshape(5, 7, 64) * s2[..., None]).reshape(5, 448)
    np.testing.assert_array_equal(dec, q)
    # relative error bounded by half an e4m3 ulp (2^-4) of the block scale grid
    assert np.all(np.abs(q - x) <= np.repeat(s, 64, axis=1) * 448.0 * 2.0 ** -4 + 1e-12)
