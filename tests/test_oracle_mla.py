"""The grouped output projection of the oracle, pinned by scipy's block-diagonal matrix and by
special cases of the inverse RoPE."""
import numpy as np
import scipy.linalg
import torch

from oracle import mla as omla


def test_o_grouped_is_block_diagonal_product():
    rng = np.random.default_rng(0)
    T, G, K, R, dim = 3, 4, 32, 16, 24
    o = rng.standard_normal((T, G * K))
    wa = rng.standard_normal((G * R, K))
    wb = rng.standard_normal((dim, G * R))
    bd = scipy.linalg.block_diag(*[wa[g * R:(g + 1) * R].T for g in range(G)])    # [G*K, G*R]
    np.testing.assert_allclose(omla.o_grouped(o, wa, wb, G, mid_bf16=False), o @ bd @ wb.T, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(omla.o_grouped(o[:, :K], wa[:R], wb[:, :R], 1, mid_bf16=False),
                               o[:, :K] @ wa[:R].T @ wb[:, :R].T, rtol=1e-12, atol=1e-12)
    # the bf16 intermediate stays within bf16 rounding of the exact product
    exact = o @ bd
    rnd = omla._bf16(exact)
    assert np.all(np.abs(rnd - exact) <= np.abs(exact) * 2.0 ** -8)


def test_o_project_special_rotations():
    rng = np.random.default_rng(1)
    T, H, D, rd, G, R, dim = 2, 4, 128, 64, 2, 16, 8
    o = torch.from_numpy(rng.standard_normal((T, H, D)).astype(np.float32))
    wa = rng.standard_normal((G * R, H * D // G))
    wb = rng.standard_normal((dim, G * R))
    cos0, sin0 = torch.ones(1, rd // 2), torch.zeros(1, rd // 2)
    pos = torch.zeros(T, dtype=torch.int32)
    np.testing.assert_array_equal(omla.o_project(o, pos, cos0, sin0, wa, wb, G),
                                  omla.o_grouped(o.reshape(T, -1).numpy(), wa, wb, G))
    # quarter turn (cos 0, sin 1), inverse: (x0, x1) -> (x1, -x0)
    cq, sq = torch.zeros(1, rd // 2), torch.ones(1, rd // 2)
    o_sw = o.clone()
    pairs = o_sw[..., D - rd:].reshape(T, H, rd // 2, 2)
    o_sw[..., D - rd:] = torch.stack([pairs[..., 1], -pairs[..., 0]], dim=-1).reshape(T, H, rd)
    np.testing.assert_array_equal(omla.o_project(o, pos, cq, sq, wa, wb, G),
                                  omla.o_grouped(o_sw.reshape(T, -1).numpy(), wa, wb, G))
