"""The lane layout of the fp4 key kernel (csrc/qat.hip rotate_fp4_kernel), modelled on the CPU.

A row of n values spans L = n / 32 lanes with E = 32 consecutive values per lane (one fp4 block
per lane).  Butterfly stages shorter than E run inside a lane; stage h >= E pairs lane l with
lane l ^ (h / E) at the same register: the lane with bit h / E clear keeps v + o, the other
o - v (the kernel's fma(+-1, v, o)).  The model runs that schedule with float32 arithmetic and
must reproduce the oracle bit for bit, signs of zero included."""
import numpy as np
import pytest

from oracle import qat


def _kernel_model(x):
    n = x.shape[-1]
    E = 32
    L = n // E
    v = x.astype(np.float32).reshape(-1, L, E).copy()        # [row, lane, register]
    h = 1
    while h < E:                                                # in-lane stages
        for i in range(E):
            if i & h:
                continue
            a, b = v[:, :, i].copy(), v[:, :, i + h].copy()
            v[:, :, i], v[:, :, i + h] = a + b, a - b
        h *= 2
    m = 1
    while m < L:                                                # cross-lane stages
        lanes = np.arange(L)
        other = v[:, lanes ^ m, :]
        up = (lanes & m).astype(bool)[None, :, None]
        v = np.where(up, other - v, v + other).astype(np.float32)
        m *= 2
    return (v.reshape(x.shape) * qat.rotate_scale(n)).astype(np.float32)


@pytest.mark.parametrize("n", [32, 64, 128, 256, 512, 1024])
def test_lane_schedule_reproduces_oracle(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((6, n)) * np.exp2(rng.integers(-10, 10, (6, n)))).astype(np.float32)
    x[0] = 0.0
    x[1] = 1.5                        # equal values: differences are +0
    got, ref = _kernel_model(x), qat.hadamard_rotate(x)
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(np.signbit(got), np.signbit(ref))
