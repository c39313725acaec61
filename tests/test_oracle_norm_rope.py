"""Pins oracle.norm_rope against the reference's goldens, closed forms and invariants."""
import math
import os

import numpy as np
import torch

from conftest import GOLDEN
from oracle import norm_rope as nr


def _g():
    return np.load(os.path.join(GOLDEN, "norm_rope.npz"))


def test_freqs_match_reference_golden_bitwise():
    g = _g()
    fy = nr.precompute_freqs_cis(64, 96, 65536, 160000.0, 16, 32, 1)
    fn = nr.precompute_freqs_cis(64, 96, 0, 10000.0, 40, 32, 1)
    np.testing.assert_array_equal(fy.real.numpy(), g["freqs_yarn_re"])
    np.testing.assert_array_equal(fy.imag.numpy(), g["freqs_yarn_im"])
    np.testing.assert_array_equal(fn.real.numpy(), g["freqs_plain_re"])
    np.testing.assert_array_equal(fn.imag.numpy(), g["freqs_plain_im"])


def test_rotary_matches_reference_golden():
    g = _g()
    fy = nr.precompute_freqs_cis(64, 96, 65536, 160000.0, 16, 32, 1)
    x3, x4 = torch.from_numpy(g["x3"]), torch.from_numpy(g["x4"])
    np.testing.assert_allclose(nr.apply_rotary_emb(x3, fy).numpy(), g["rope3"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(nr.apply_rotary_emb(x3, fy, inverse=True).numpy(), g["rope3_inv"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(nr.apply_rotary_emb(x4, fy).numpy(), g["rope4"], rtol=0, atol=1e-6)


def test_rmsnorm_golden_and_closed_form():
    g = _g()
    x, w = torch.from_numpy(g["rms_x"]), torch.from_numpy(g["rms_w"])
    np.testing.assert_allclose(nr.rmsnorm(x, w).numpy(), g["rms_out"], rtol=1e-6, atol=1e-7)
    xd = x.double()
    ref = w.double() * xd / torch.sqrt((xd ** 2).mean(-1, keepdim=True) + 1e-6)
    np.testing.assert_allclose(nr.rmsnorm(x, w).double().numpy(), ref.numpy(), rtol=2e-6)


def test_yarn_correction_range_closed_form():
    assert nr.yarn_correction_range(64, 160000.0, 65536, 32, 1) == (15, 25)
    # hand formula: dim*ln(L/(2*pi*beta))/(2 ln base)
    lo = 64 * math.log(65536 / (32 * 2 * math.pi)) / (2 * math.log(160000.0))
    hi = 64 * math.log(65536 / (1 * 2 * math.pi)) / (2 * math.log(160000.0))
    assert (math.floor(lo), math.ceil(hi)) == (15, 25)


def test_no_yarn_is_plain_geometric():
    f = nr.precompute_freqs(64, 1, 0, 10000.0, 40, 32, 1)
    ref = 10000.0 ** (-np.arange(0, 64, 2) / 64.0)
    np.testing.assert_allclose(f.numpy(), ref, rtol=2e-6)
    # YaRN: dims below `low` keep full frequency/factor, above `high` keep the raw frequency
    fy = nr.precompute_freqs(64, 1, 65536, 160000.0, 16, 32, 1).double().numpy()
    raw = 160000.0 ** (-np.arange(0, 64, 2) / 64.0)
    np.testing.assert_allclose(fy[:15], raw[:15], rtol=2e-6)
    np.testing.assert_allclose(fy[25:], raw[25:] / 16, rtol=2e-6)


def test_rotation_preserves_pair_norm_and_inverts():
    torch.manual_seed(0)
    x = torch.randn(1, 40, 64)
    f = nr.precompute_freqs_cis(64, 40, 65536, 160000.0, 16, 32, 1)
    y = nr.apply_rotary_emb(x, f)
    n0 = x.reshape(1, 40, 32, 2).norm(dim=-1)
    n1 = y.reshape(1, 40, 32, 2).norm(dim=-1)
    np.testing.assert_allclose(n0.numpy(), n1.numpy(), rtol=1e-5)
    z = nr.apply_rotary_emb(y, f, inverse=True)
    np.testing.assert_allclose(z.numpy(), x.numpy(), atol=1e-5)
    # position 0 is the identity
    np.testing.assert_array_equal(y[0, 0].numpy(), x[0, 0].numpy())
