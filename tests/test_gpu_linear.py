"""GPU parity of the decode projections: smla_linear, smla_rope and smla_o_proj.

* ``smla_rope`` equals the oracle's float32 rotation (golden-pinned) bit for bit, forward and
  inverse, bf16 and fp32.
* ``smla_linear`` equals the float64 product of the same bf16 operands within the float32
  accumulation error (1e-5 of sum |x||w|, far below what a dropped K slice or a wrong row would
  change), plus half a bf16 ulp when the output is bf16; with fp32 operands (the tiled GEMM only)
  within (K + 8) 2^-23 of sum |x||w|, twice the textbook bound of a K-term fp32 dot product.
  Up to 32 bf16 rows run the weight-streaming kernel, other shapes the tiled MFMA GEMM
  (ragged token and output tiles, K tails, groups, fp32 operands).
* ``smla_o_proj`` with the fused inverse RoPE equals, bit for bit, the standalone inverse rotation
  followed by the unrotated projection, and the oracle's o_project within bf16 tolerance.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import mla as omla
from oracle import norm_rope as onr

pytestmark = pytest.mark.gpu


def _check_linear(got, x, w, G, out_dtype):
    x64, w64 = x.double().numpy(), w.double().numpy()
    T, GK = x64.shape
    K = GK // G
    N = w64.shape[0] // G
    ref = np.concatenate([x64[:, g * K:(g + 1) * K] @ w64[g * N:(g + 1) * N].T for g in range(G)], axis=1)
    mag = np.concatenate([np.abs(x64[:, g * K:(g + 1) * K]) @ np.abs(w64[g * N:(g + 1) * N]).T for g in range(G)],
                         axis=1)
    acc_tol = (K + 8) * 2.0 ** -23 if x.dtype == torch.float32 else 1e-5
    tol = acc_tol * mag + (np.abs(ref) * 2.0 ** -8 if out_dtype == torch.bfloat16 else 0.0)
    err = np.abs(got.double().cpu().numpy() - ref)
    assert np.all(err <= tol), f"max err {err.max():.3e}, worst ratio {(err / np.maximum(tol, 1e-30)).max():.3f}"


@pytest.mark.parametrize("T,G,N,K,out_dtype", [
    (8, 8, 1024, 4096, torch.bfloat16),      # o_grouped's grouped product at decode (LDS form)
    (12, 8, 1024, 4096, torch.bfloat16),     # the same width in the register form (T > 8)
    (8, 1, 4096, 8192, torch.float32),       # its second product (8 waves x 16 steps)
    (9, 1, 4096, 8192, torch.float32),       # register form
    (1, 1, 256, 4096, torch.float32),
    (3, 2, 48, 512, torch.float32),          # one wave per workgroup
    (16, 2, 64, 1024, torch.bfloat16),       # short K slices: the guarded last batch
    (17, 1, 128, 512, torch.float32),        # two token tiles, one ragged
    (32, 4, 32, 2048, torch.bfloat16),
    # the LDS form over 8192 rows: 2 and 4 waves, one wave with K = 512
    (5, 1, 8192, 1024, torch.float32),
    (8, 4, 2048, 2048, torch.bfloat16),
    (2, 1, 8192, 512, torch.float32),
    # the tiled MFMA GEMM
    (768, 1, 21760, 512, torch.float32),       # 256 x 256 DMA tiles: 3 x 85 of them
    (520, 2, 11000, 576, torch.bfloat16),      # the same, ragged tokens and outputs, two groups
    (64, 1, 1024, 4096, torch.float32),
    (4096, 1, 1024, 4096, torch.bfloat16),     # prefill's q_down
    (300, 1, 200, 520, torch.float32),         # ragged token and output tiles, a K tail
    (100, 8, 1024, 4096, torch.bfloat16),      # o_grouped's grouped product at prefill
    (33, 2, 48, 24, torch.float32),            # K shorter than one step
])
@pytest.mark.parametrize("operands", [torch.bfloat16, torch.float32])
def test_linear_vs_fp64(dev, T, G, N, K, out_dtype, operands):
    from smla import ops
    announce(f"linear T={T} G={G} N={N} K={K} out={out_dtype} operands={operands}")
    g = torch.Generator().manual_seed(T * 7 + G + N + K)
    x = torch.randn(T, G * K, generator=g).to(operands)
    w = (torch.randn(G * N, K, generator=g) * 0.05).to(operands)
    y = ops.linear_op(x.to(dev), w.to(dev), G, out_dtype)
    torch.cuda.synchronize()
    assert y.dtype == out_dtype and y.shape == (T, G * N)
    _check_linear(y.float(), x, w, G, out_dtype)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("inverse", [False, True])
def test_rope_bit_exact(dev, dt, inverse):
    from smla import norm_rope as snr
    from smla import ops
    announce(f"rope dtype={dt} inverse={inverse}")
    g = torch.Generator().manual_seed(2)
    T, H, D, rd = 9, 64, 512, 64
    x = torch.randn(T, H, D, generator=g).to(dt)
    pos = torch.randint(0, 65536, (T,), generator=g, dtype=torch.int32)
    pos[0] = 0
    cos_t, sin_t = snr.rope_tables(rd, 65536, device=dev)
    got = x.to(dev)
    ops.rope_op_(got, pos.to(dev), cos_t, sin_t, inverse)
    cis = torch.complex(cos_t.cpu()[pos.long()], sin_t.cpu()[pos.long()])
    ref = x.clone()
    ref[..., D - rd:] = onr.apply_rotary_emb(x[None, :, :, D - rd:], cis, inverse=inverse)[0]
    assert torch.equal(got.cpu(), ref)


@pytest.mark.parametrize("T", [1, 8, 20, 40, 300])
def test_o_proj_fused_rope(dev, T):
    from smla import norm_rope as snr
    from smla import ops
    announce(f"o_proj T={T}")
    g = torch.Generator().manual_seed(T)
    H, D, rd, G, R, dim = 64, 512, 64, 8, 1024, 4096
    o = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    wa = (torch.randn(G * R, H * D // G, generator=g) * 0.02).to(torch.bfloat16)
    wb = (torch.randn(dim, G * R, generator=g) * 0.02).to(torch.bfloat16)
    pos = torch.randint(0, 65536, (T,), generator=g, dtype=torch.int32)
    cos_t, sin_t = snr.rope_tables(rd, 65536, device=dev)
    od, wad, wbd, posd = o.to(dev), wa.to(dev), wb.to(dev), pos.to(dev)
    fused = ops.o_proj_op(od, posd, cos_t, sin_t, wad, wbd, G, torch.float32)
    # the same rotation done first by the standalone kernel: identical operands, identical result
    rot = od.clone()
    ops.rope_op_(rot, posd, cos_t, sin_t, True)
    two = ops.o_proj_op(rot, None, None, None, wad, wbd, G, torch.float32)
    assert torch.equal(fused, two)
    # against the oracle (float64 products, bf16 intermediate)
    ref = omla.o_project(o, pos, cos_t.cpu(), sin_t.cpu(), wa.float().numpy(), wb.float().numpy(), G)
    np.testing.assert_allclose(fused.cpu().double().numpy(), ref, rtol=1e-2, atol=2e-2 * np.abs(ref).max())


@pytest.mark.parametrize("T", [600, 2048])
def test_o_proj_fused_rope_wide(dev, T):
    """The grouped product on the DMA tiles (600 tokens: 128 x 128, 2048: 256 x 256) with the
    inverse RoPE applied in LDS: equal to the standalone rotation followed by the plain product bit
    for bit, and to the oracle on a sample of tokens (each token's output depends on that token
    alone)."""
    from smla import norm_rope as snr
    from smla import ops
    announce(f"o_proj T={T} (DMA tiles with RoPE)")
    g = torch.Generator().manual_seed(T)
    H, D, rd, G, R, dim = 64, 512, 64, 8, 1024, 4096
    o = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    wa = (torch.randn(G * R, H * D // G, generator=g) * 0.02).to(torch.bfloat16)
    wb = (torch.randn(dim, G * R, generator=g) * 0.02).to(torch.bfloat16)
    pos = torch.randint(0, 65536, (T,), generator=g, dtype=torch.int32)
    cos_t, sin_t = snr.rope_tables(rd, 65536, device=dev)
    od, wad, wbd, posd = o.to(dev), wa.to(dev), wb.to(dev), pos.to(dev)
    fused = ops.o_proj_op(od, posd, cos_t, sin_t, wad, wbd, G, torch.float32)
    rot = od.clone()
    ops.rope_op_(rot, posd, cos_t, sin_t, True)
    two = ops.o_proj_op(rot, None, None, None, wad, wbd, G, torch.float32)
    assert torch.equal(fused, two)
    idx = torch.tensor([0, 1, 127, 128, 255, 256, T // 2, T - 2, T - 1])
    ref = omla.o_project(o[idx], pos[idx], cos_t.cpu(), sin_t.cpu(), wa.float().numpy(), wb.float().numpy(), G)
    np.testing.assert_allclose(fused.cpu()[idx].double().numpy(), ref, rtol=1e-2, atol=2e-2 * np.abs(ref).max())


def test_mla_mirror_routes(dev):
    """mla.linear / o_grouped / o_project run the weight-streaming kernels at decode shapes and the
    tiled GEMM beyond; both agree with the oracle."""
    from smla import mla
    from smla import norm_rope as snr
    announce("mla mirror")
    g = torch.Generator().manual_seed(5)
    H, D, G, R, dim = 64, 512, 8, 1024, 4096
    wa = (torch.randn(G * R, H * D // G, generator=g) * 0.02).to(torch.bfloat16)
    wb = (torch.randn(dim, G * R, generator=g) * 0.02).to(torch.bfloat16)
    cos_t, sin_t = snr.rope_tables(64, 65536, device=dev)
    for T in (4, 40):                  # decode kernel, then the GEMM path
        o = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
        pos = torch.randint(0, 65536, (T,), generator=g, dtype=torch.int32)
        y = mla.o_project(o.to(dev), pos.to(dev), cos_t, sin_t, wa.to(dev), wb.to(dev))
        ref = omla.o_project(o, pos, cos_t.cpu(), sin_t.cpu(), wa.float().numpy(), wb.float().numpy(), G)
        np.testing.assert_allclose(y.cpu().double().numpy(), ref, rtol=2e-2, atol=2e-2 * np.abs(ref).max())
    x = torch.randn(3, 4096, generator=g).to(torch.bfloat16)
    W = (torch.randn(1024, 4096, generator=g) * 0.02).to(torch.bfloat16)
    y = mla.linear(x.to(dev), W.to(dev))
    np.testing.assert_allclose(y.cpu().double().numpy(), omla.linear(x.float().numpy(), W.float().numpy()),
                               rtol=2e-2, atol=2e-2)


def test_o_proj_graph_replays(dev):
    """The fused output path captured in a HIP graph: every replay, with eager work and
    synchronisations between replays, equals the eager result bit for bit."""
    from smla import norm_rope as snr
    from smla import ops
    announce("o_proj graph replay")
    g = torch.Generator().manual_seed(12)
    T, H, D, G, R, dim = 8, 64, 512, 8, 1024, 4096
    o = torch.randn(T, H, D, generator=g).to(torch.bfloat16).to(dev)
    wa = (torch.randn(G * R, H * D // G, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    wb = (torch.randn(dim, G * R, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    pos = torch.randint(0, 65536, (T,), generator=g, dtype=torch.int32).to(dev)
    cos_t, sin_t = snr.rope_tables(64, 65536, device=dev)
    eager = ops.o_proj_op(o, pos, cos_t, sin_t, wa, wb, G, torch.bfloat16)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ops.o_proj_op(o, pos, cos_t, sin_t, wa, wb, G, torch.bfloat16)
    for r in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"
        ops.o_proj_op(o, pos, cos_t, sin_t, wa, wb, G, torch.bfloat16)     # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("shape,dt", [((2, 5, 64), torch.float32), ((2, 5, 8, 64), torch.bfloat16),
                                      ((1, 7, 64, 64), torch.float32)])
@pytest.mark.parametrize("inverse", [False, True])
def test_apply_rotary_emb_mirror(dev, shape, dt, inverse):
    """smla.norm_rope.apply_rotary_emb (ref_torch/norm_rope.py:53-62 signature, on smla_rope) equals
    the oracle's rotation bit for bit."""
    from smla import norm_rope as snr
    announce(f"apply_rotary_emb {shape} {dt} inverse={inverse}")
    g = torch.Generator().manual_seed(sum(shape))
    x = torch.randn(*shape, generator=g).to(dt)
    cis = onr.precompute_freqs_cis(shape[-1], shape[1], 65536, 160000.0, 16, 32, 1)
    got = snr.apply_rotary_emb(x.to(dev), cis.to(dev), inverse=inverse).cpu()
    ref = onr.apply_rotary_emb(x, cis, inverse=inverse)
    assert got.dtype == x.dtype and torch.equal(got, ref)
