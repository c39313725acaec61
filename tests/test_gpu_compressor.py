"""GPU parity of the compressor kernels: block mean pool (bit-exact), gated pool / compressor_prefill
(reference goldens + oracle), the device ring (oracle ring), fp8 quantisation (bit-exact)."""
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN, announce
from oracle import compressor as oc
from oracle import fp8 as ofp8
from oracle import norm_rope as onr

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dt,B,N,D", [(torch.bfloat16, 2, 64, 576), (torch.float32, 1, 40, 512),
                                      (torch.bfloat16, 8, 32768, 576)])
def test_block_mean_pool_bit_exact(dev, dt, B, N, D):
    from smla import compressor as sc
    announce(f"mean pool {dt} B={B} N={N}")
    g = torch.Generator().manual_seed(N)
    x = (torch.randn(B, N, D, generator=g) * 0.05).to(dt)
    got = sc.block_mean_pool(x.to(dev), 4).cpu()
    ref = oc.mean_pool(x, 4).to(dt)
    assert torch.equal(got, ref)


def test_compressor_prefill_matches_reference_golden(dev):
    from smla import compressor as sc
    announce("compressor_prefill golden")
    g = np.load(os.path.join(GOLDEN, "compressor.npz"))
    t = {k.split("__", 1)[1]: torch.from_numpy(g[k]) for k in g.files if k.startswith("wide_rem__")}
    kv, state = sc.compressor_prefill(t["x"].to(dev), t["wkv"].to(dev), t["wgate"].to(dev), t["ape"].to(dev),
                                      t["norm_w"].to(dev), head_dim=512, ratio=4, rope_head_dim=64)
    np.testing.assert_allclose(kv.cpu().numpy(), t["kv"].numpy(), rtol=1e-4, atol=2e-5)
    for key in ("kv", "score", "kv_rem"):
        np.testing.assert_allclose(state[key].cpu().numpy(), t["state_" + key].numpy(), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("fp8_sim", [False, True])
def test_gated_pool_vs_oracle(dev, fp8_sim):
    from smla import ops
    announce(f"gated pool fp8_sim={fp8_sim}")
    g = torch.Generator().manual_seed(5)
    B, N, d, r, rd = 2, 64, 512, 4, 64
    kv = torch.randn(B, N, 2 * d, generator=g)
    sc_ = torch.randn(B, N, 2 * d, generator=g) * 2
    ape = torch.randn(r, 2 * d, generator=g)
    nw = 1 + 0.1 * torch.randn(d, generator=g)
    cis = onr.precompute_freqs_cis(rd, N, 65536, 160000.0, 16, 32, 1)
    cos_t, sin_t = cis.real.contiguous(), cis.imag.contiguous()
    got = ops.gated_pool_op(kv.to(dev), sc_.to(dev), ape.to(dev), nw.to(dev), cos_t.to(dev), sin_t.to(dev), r, rd,
                            1e-6, int(fp8_sim)).cpu()
    ref = oc.gated_pool(kv, sc_, ape, nw, cis, r, rd)
    if not fp8_sim:
        np.testing.assert_allclose(got.numpy(), ref.numpy(), rtol=1e-4, atol=2e-5)
    else:
        nope_ref, s = ofp8.act_quant_sim(ref[..., : d - rd].numpy(), 64)
        np.testing.assert_allclose(got[..., d - rd:].numpy(), ref[..., d - rd:].numpy(), rtol=1e-4, atol=2e-5)
        # fp8 round trip of values that agree to ~1e-6: at most one e4m3 step apart, rarely
        step = np.repeat(s, 64, axis=-1) * 448.0 * 2.0 ** -3
        diff = np.abs(got[..., : d - rd].numpy() - nope_ref)
        assert np.all(diff <= step + 1e-7)
        assert (diff > 1e-7).mean() < 1e-3


@pytest.mark.parametrize("fp8_sim", [False, True])
def test_ring_vs_oracle_ring(dev, fp8_sim):
    from smla import compressor as sc
    announce(f"ring step fp8_sim={fp8_sim}")
    g = torch.Generator().manual_seed(6)
    B, d, r, rd, n_pre, n = 2, 512, 4, 64, 10, 30
    kvp = torch.randn(B, n, 2 * d, generator=g)
    scp = torch.randn(B, n, 2 * d, generator=g)
    ape = torch.randn(r, 2 * d, generator=g)
    nw = 1 + 0.1 * torch.randn(d, generator=g)
    ring = sc.Ring(B, d, ape, nw, ratio=r, rope_head_dim=rd, max_pos=4096, fp8_sim=fp8_sim, device=dev)
    ring.init_from_prefill(kvp[:, :n_pre].to(dev), scp[:, :n_pre].to(dev))
    cap = n // r
    comp = torch.zeros(B, cap, d, device=dev)
    for p in range(n_pre, n):
        ring.step(kvp[:, p].to(dev), scp[:, p].to(dev), torch.full((B,), p, dtype=torch.int32, device=dev), comp)
    comp = comp.cpu()
    freqs = onr.precompute_freqs(rd, 4096, 65536, 160000.0, 16, 32, 1)
    for b in range(B):
        kvs, scs = oc.ring_init(kvp[b, :n_pre], scp[b, :n_pre], ape, r)
        for p in range(n_pre, n):
            row = oc.ring_step(kvs, scs, kvp[b, p], scp[b, p], p, ape, nw, freqs, r, rd, fp8_sim=fp8_sim)
            if row is None:
                continue
            grp = (p + 1) // r - 1
            got = comp[b, grp]
            np.testing.assert_allclose(got[d - rd:].numpy(), row[d - rd:].numpy(), rtol=1e-4, atol=2e-5)
            if fp8_sim:
                diff = (got[: d - rd] - row[: d - rd]).abs()
                assert (diff > 1e-7).float().mean().item() < 0.02
                assert diff.max().item() <= row[: d - rd].abs().max().item() * 0.13
            else:
                np.testing.assert_allclose(got.numpy(), row.numpy(), rtol=1e-4, atol=2e-5)
        # the ring itself (moves and the score + ape adds only): bit for bit
        assert torch.equal(ring.ring_kv[b].cpu(), kvs) and torch.equal(ring.ring_sc[b].cpu(), scs)


def test_ring_step_kv_equals_separate_calls(dev):
    """smla_ring_step_kv (the kv row's epilogue and the ring step in one launch) against
    smla_row_epilogue then smla_ring_step on the same inputs: ring state, compressed rows and
    window-cache rows bit for bit, over steps that emit and steps that do not, with one sequence
    at a negative position (left untouched by both)."""
    from smla import _lib, ops
    from smla import compressor as sc
    announce("ring step + kv row epilogue in one launch")
    g = torch.Generator().manual_seed(11)
    B, d, r, rd, rows = 3, 512, 4, 64, 64
    ape = torch.randn(r, 2 * d, generator=g)
    nw = 1 + 0.1 * torch.randn(d, generator=g)
    kvn = (1 + 0.1 * torch.randn(d, generator=g)).to(dev)
    pre_kv, pre_sc = torch.randn(B, 6, 2 * d, generator=g), torch.randn(B, 6, 2 * d, generator=g)
    rings, comps, caches = [], [], []
    for _ in range(2):
        ring = sc.Ring(B, d, ape, nw, ratio=r, rope_head_dim=rd, max_pos=4096, fp8_sim=True, device=dev)
        ring.init_from_prefill(pre_kv.to(dev), pre_sc.to(dev))
        rings.append(ring)
        comps.append(torch.zeros(B, 16, d, device=dev))
        caches.append(torch.zeros(B, rows, d, dtype=torch.bfloat16, device=dev))
    cos_t, sin_t = rings[0].cos_t, rings[0].sin_t
    for p in range(6, 16):
        y = torch.randn(B, 5 * d, generator=g).to(dev)        # [kv row | kv proj | score proj], one projection
        kv_x, kvp, scp = y[:, :d], y[:, d:3 * d], y[:, 3 * d:]
        pos = torch.tensor([p, p + 1, -1 if p == 9 else p + 2], dtype=torch.int32, device=dev)
        ops.row_epilogue(kv_x, kvn, pos, cos_t, sin_t, rd, _lib.SIM_FP8, caches[0], cache_rows=rows)
        rings[0].step(kvp, scp, pos, comps[0])
        ops.ring_step_kv(rings[1], kvp, scp, pos, comps[1], kv_x, kvn, cos_t, sin_t, rd, _lib.SIM_FP8, caches[1])
    torch.cuda.synchronize()
    assert torch.equal(rings[0].ring_kv, rings[1].ring_kv) and torch.equal(rings[0].ring_sc, rings[1].ring_sc)
    assert torch.equal(comps[0], comps[1])
    assert torch.equal(caches[0].view(torch.int16), caches[1].view(torch.int16))
    assert comps[0].abs().sum() > 0 and caches[0].float().abs().sum() > 0   # rows were written


def test_quant_fp8_encoder_every_code(dev):
    """The quantiser's e4m3 encoding on the device over every finite e4m3 value, every midpoint
    between neighbours and the floats next to each midpoint, tiny values, signed zeros and random
    values: blocks that open with 448 have scale 1, so their codes are the plain encoding."""
    from smla import ops
    announce("quant fp8 encoder")
    ref = ofp8.e4m3_decode(np.arange(256, dtype=np.uint8))
    vals = ref[np.isfinite(ref)]
    pos = np.unique(np.abs(vals))
    mids = ((pos[1:].astype(np.float64) + pos[:-1]) / 2).astype(np.float32)
    rnd = np.clip(np.random.default_rng(5).standard_normal(4000).astype(np.float32) * 50, -448, 448)
    x = np.concatenate([vals, mids, -mids, np.nextafter(mids, 0), np.nextafter(mids, 1),
                        np.nextafter(-mids, 0), np.nextafter(-mids, -1), rnd,
                        np.float32([2.0 ** -10, -(2.0 ** -10), 3 * 2.0 ** -10, 1e-30, -1e-30, 0.0, -0.0,
                                    2.0 ** -9, 448.0, -448.0])]).astype(np.float32)
    nb = (x.size + 62) // 63
    blocks = np.zeros((nb, 64), dtype=np.float32)
    blocks[:, 0] = 448.0
    blocks[:, 1:].flat[:x.size] = x
    codes, scales = ops.quant_fp8_pow2_op(torch.from_numpy(blocks).to(dev))
    assert torch.all(scales.cpu() == 1.0)
    got = codes.cpu().numpy().reshape(nb, 64)[:, 1:].reshape(-1)[:x.size]
    np.testing.assert_array_equal(got, ofp8.e4m3_encode(x).astype(np.uint8))


def test_quant_fp8_bit_exact(dev):
    from smla import ops
    announce("quant fp8")
    g = torch.Generator().manual_seed(8)
    x = torch.randn(300, 576, generator=g) * torch.exp2(torch.randint(-12, 8, (300, 1), generator=g).float())
    x[0] = 0
    x[1, :64] = 448.0 * 2.0 ** 3           # exact power-of-two block
    x[2, 5] = -1e-6
    codes, scales = ops.quant_fp8_pow2_op(x.to(dev))
    rc, rs = ofp8.quantize_e4m3_pow2(x.numpy(), 64)
    np.testing.assert_array_equal(scales.cpu().numpy(), rs)
    np.testing.assert_array_equal(codes.cpu().numpy(), rc)
    codes_b, scales_b = ops.quant_fp8_pow2_op(x.to(torch.bfloat16).to(dev))
    rc_b, rs_b = ofp8.quantize_e4m3_pow2(x.to(torch.bfloat16).float().numpy(), 64)
    np.testing.assert_array_equal(codes_b.cpu().numpy(), rc_b)
    np.testing.assert_array_equal(scales_b.cpu().numpy(), rs_b)
