"""GPU parity of the indexer-key transform (smla_rotate_fp4) and of the compressor's rotate mode.

The standalone kernel must equal the oracle (``oracle/qat.py``) bit for bit: the rotation alone,
the fp4 round trip alone, both, and the stored form (packed codes and ue8m0 scales), for every
supported row length, fp32 and bf16 inputs, a ragged row count, and blocks that reach the edge
cases (all zeros, subnormal values under the amax floor, values on e2m1 midpoints, exact powers of
two).  The compressor with ``rotate`` must equal the standalone kernel applied to its unquantised
output, bit for bit, and the oracle's pooling followed by the oracle's transform up to the rare
fp4 code flip that a 1e-6 difference before quantisation can cause."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import compressor as oc
from oracle import norm_rope as onr
from oracle import qat as oqat

pytestmark = pytest.mark.gpu

NS = [32, 64, 128, 256, 512, 1024]


def _inputs(n, rows, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, n, generator=g) * torch.exp2(torch.randint(-20, 20, (rows, 1), generator=g).float())
    x[0] = 0.0                                        # amax floor, every code zero
    x[1] = 1e-40                                      # subnormal inputs under the floor
    if n >= 64:
        # a block of e2m1 midpoints (times a power of two) and one exact power of two
        mids = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0])
        x[2, :32] = mids.repeat(4) * 2.0 ** 7 * torch.where(torch.arange(32) % 3 == 0, -1.0, 1.0)
        x[2, 32:64] = 2.0 ** -3
    return x


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("n", NS)
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_rotate_fp4_bit_exact(dev, n, dt):
    from smla import qat as sq
    rows = 37
    announce(f"rotate_fp4 n={n} dtype={dt} rows={rows}")
    x = _inputs(n, rows, n).to(dt)
    xf = x.float().numpy()
    xd = x.to(dev)
    rot = oqat.hadamard_rotate(xf)
    # bit patterns: signs of zero included
    np.testing.assert_array_equal(_bits(sq.hadamard_rotate(xd).cpu().numpy()), _bits(rot))
    np.testing.assert_array_equal(_bits(sq.fp4_act_quant(xd).cpu().numpy()), _bits(oqat.fp4_act_quant(xf)))
    np.testing.assert_array_equal(_bits(sq.rotate_fp4(xd).cpu().numpy()), _bits(oqat.rotate_fp4(xf)))
    codes, scales = sq.fp4_pack(xd)
    rc, rs = oqat.fp4_quantize(rot)
    np.testing.assert_array_equal(codes.cpu().numpy(), rc)
    np.testing.assert_array_equal(scales.cpu().numpy(), rs)
    codes0, scales0 = sq.fp4_pack(xd, rotate=False)
    rc0, rs0 = oqat.fp4_quantize(xf)
    np.testing.assert_array_equal(codes0.cpu().numpy(), rc0)
    np.testing.assert_array_equal(scales0.cpu().numpy(), rs0)


def test_rotate_fp4_large_batch(dev):
    """The bench shape: 65536 keys of 128 dims, stored form and round trip in one launch."""
    from smla import ops
    announce("rotate_fp4 [65536,128]")
    g = torch.Generator().manual_seed(11)
    x = torch.randn(65536, 128, generator=g)
    out, codes, scales = ops.rotate_fp4_op(x.to(dev), True, True, True, True)
    ref = oqat.rotate_fp4(x.numpy())
    np.testing.assert_array_equal(_bits(out.cpu().numpy()), _bits(ref))
    rc, rs = oqat.fp4_quantize(oqat.hadamard_rotate(x.numpy()))
    np.testing.assert_array_equal(codes.cpu().numpy(), rc)
    np.testing.assert_array_equal(scales.cpu().numpy(), rs)
    np.testing.assert_array_equal(oqat.fp4_dequantize(codes.cpu().numpy(), scales.cpu().numpy()), ref)


def _pool_case(d, seed):
    g = torch.Generator().manual_seed(seed)
    B, N, r, rd = 2, 64, 4, 64
    kv = torch.randn(B, N, 2 * d, generator=g)
    sc_ = torch.randn(B, N, 2 * d, generator=g) * 2
    ape = torch.randn(r, 2 * d, generator=g)
    nw = 1 + 0.1 * torch.randn(d, generator=g)
    cis = onr.precompute_freqs_cis(rd, N, 65536, 160000.0, 16, 32, 1)
    return kv, sc_, ape, nw, cis, r, rd


@pytest.mark.parametrize("d", [128, 256, 512])
def test_gated_pool_rotate_fp4(dev, d):
    from smla import _lib, ops
    from smla import qat as sq
    announce(f"gated pool rotate d={d}")
    kv, sc_, ape, nw, cis, r, rd = _pool_case(d, d)
    cos_t, sin_t = cis.real.contiguous().to(dev), cis.imag.contiguous().to(dev)
    args = (kv.to(dev), sc_.to(dev), ape.to(dev), nw.to(dev), cos_t, sin_t, r, rd, 1e-6)
    plain = ops.gated_pool_op(*args, _lib.SIM_NONE)
    fused = ops.gated_pool_op(*args, _lib.SIM_ROTATE_FP4)
    # the fused epilogue equals the standalone transform of the unquantised rows
    np.testing.assert_array_equal(fused.cpu().numpy(), sq.rotate_fp4(plain).cpu().numpy())
    # and the oracle's pooling + transform, up to rare one-step code flips
    ref = oqat.rotate_fp4(oc.gated_pool(kv, sc_, ape, nw, cis, r, rd).numpy())
    got = fused.cpu().numpy()
    _, s = oqat.fp4_quantize(ref)
    step = np.repeat(np.exp2(s.astype(np.int64) - 127), 32, axis=-1) * 2.0
    diff = np.abs(got - ref)
    assert np.all(diff <= step)
    assert (diff > 0).mean() < 0.01


def test_ring_rotate_matches_prefill_pool(dev):
    """The decode ring with the rotate mode emits the rows the prefill pool computes, bit for bit."""
    from smla import _lib, ops
    from smla import compressor as sc
    announce("ring rotate vs prefill pool")
    d = 128
    kv, sc_, ape, nw, cis, r, rd = _pool_case(d, 9)
    B, N = kv.shape[:2]
    n_pre = 10
    ring = sc.Ring(B, d, ape, nw, ratio=r, rope_head_dim=rd, max_pos=N, fp8_sim=False, device=dev, rotate=True)
    ring.init_from_prefill(kv[:, :n_pre].to(dev), sc_[:, :n_pre].to(dev))
    comp = torch.zeros(B, N // r, d, device=dev)
    for p in range(n_pre, N):
        ring.step(kv[:, p].to(dev), sc_[:, p].to(dev), torch.full((B,), p, dtype=torch.int32, device=dev), comp)
    pool = ops.gated_pool_op(kv.to(dev), sc_.to(dev), ape.to(dev), nw.to(dev), ring.cos_t, ring.sin_t, r, rd, 1e-6,
                             _lib.SIM_ROTATE_FP4)
    first = n_pre // r                                # the first group the ring emits itself
    np.testing.assert_array_equal(comp[:, first:].cpu().numpy(), pool[:, first:].cpu().numpy())
