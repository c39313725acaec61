"""GPU parity of the decode layer's row kernels (``oracle/decode_engine.py:78-84,110-114``):

* ``smla_row_epilogue`` against the oracle's RMSNorm (``ref_torch/norm_rope.py:10-16``), RoPE
  (``:53-62``) and fp8 round trip (``v4mlx/compressor.py:11-20``): the rope channels within float32
  rounding plus half a bf16 ulp; the fp8 channels equal the oracle's except where the float32
  norm's summation order moves a value across an e4m3 rounding boundary (at most 2 % of them, each
  by one e4m3 step);
* ``smla_decode_ids`` equal, id for id, to a brute-force enumeration, and an emitted compressed
  row copied to bf16 bit for bit.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import fp8 as ofp8
from oracle import norm_rope as onr

pytestmark = pytest.mark.gpu

YARN = (65536, 160000.0, 16, 32, 1)


def _rope_ref(x, cos, sin, p):
    cis = torch.complex(cos[p:p + 1], sin[p:p + 1])
    return onr.apply_rotary_emb(x.reshape(1, 1, -1, 64), cis).reshape(x.shape)


def _bf16(t):
    return t.to(torch.bfloat16).float()


def test_kv_rows_into_cache(dev):
    from smla import _lib, ops
    from smla import norm_rope as snr
    announce("row_epilogue kv -> cache")
    g = torch.Generator().manual_seed(21)
    B, d, rows = 3, 512, 400
    x = torch.randn(B, d, generator=g) * 3
    w = 1 + 0.1 * torch.randn(d, generator=g)
    pos = torch.tensor([0, 77, 399], dtype=torch.int32)
    cos, sin = onr.rope_cos_sin(64, rows, *YARN)
    cos_d, sin_d = snr.rope_tables(64, rows, *YARN, device=dev)
    cache = torch.zeros(B, rows, d, dtype=torch.bfloat16, device=dev)
    ops.row_epilogue(x.to(dev), w.to(dev), pos.to(dev), cos_d, sin_d, 64, _lib.SIM_FP8, cache, cache_rows=rows)
    got = cache.float().cpu()
    flips = 0
    for b in range(B):
        p = int(pos[b])
        y = onr.rmsnorm(x[b], w)
        rope = _rope_ref(y[-64:], cos, sin, p)
        nope, scl = ofp8.act_quant_sim(y[:-64].numpy()[None], 64)
        row = got[b, p]
        assert torch.allclose(row[-64:], rope, rtol=2.0 ** -8, atol=1e-6)
        ref8 = torch.from_numpy(nope[0])
        diff = (row[:-64] - _bf16(ref8)).abs()
        step = torch.from_numpy(np.repeat(scl[0], 64)) * 2.0 ** (torch.floor(torch.log2(ref8.abs().clamp(min=2 ** -6))) - 3)
        assert torch.all(diff <= step * 1.01 + 1e-7), "an fp8 value off by more than one e4m3 step"
        flips += int((diff > 0).sum())
        others = torch.ones(rows, dtype=torch.bool)
        others[p] = False
        assert torch.all(got[b][others] == 0), "rows other than pos were written"
    assert flips <= 0.02 * B * 448


@pytest.mark.parametrize("B", [1, 5])
def test_q_heads_weightless_norm_and_rope(dev, B):
    from smla import _lib, ops
    from smla import norm_rope as snr
    announce(f"row_epilogue q heads B={B}")
    g = torch.Generator().manual_seed(B)
    x = torch.randn(B, 64, 512, generator=g) * 0.7
    pos = torch.randint(0, 1000, (B,), generator=g, dtype=torch.int32)
    cos, sin = onr.rope_cos_sin(64, 1000, *YARN)
    cos_d, sin_d = snr.rope_tables(64, 1000, *YARN, device=dev)
    out = torch.empty(B, 64, 512, dtype=torch.bfloat16, device=dev)
    ops.row_epilogue(x.to(dev).view(B * 64, 512), None, pos.to(dev), cos_d, sin_d, 64, _lib.SIM_NONE, out,
                     rows_per_pos=64)
    got = out.float().cpu()
    for b in range(B):
        q = x[b] * torch.rsqrt(x[b].pow(2).mean(-1, keepdim=True) + 1e-6)
        q = torch.cat([q[:, :-64], _rope_ref(q[:, -64:], cos, sin, int(pos[b]))], dim=-1)
        assert torch.allclose(got[b], q, rtol=2.0 ** -8, atol=1e-6)


def test_q_a_norm_d1024(dev):
    from smla import _lib, ops
    announce("row_epilogue q_a d=1024")
    g = torch.Generator().manual_seed(4)
    x = torch.randn(6, 1024, generator=g) * 2
    w = 1 + 0.1 * torch.randn(1024, generator=g)
    out = torch.empty(6, 1024, device=dev)
    ops.row_epilogue(x.to(dev), w.to(dev), None, None, None, 0, _lib.SIM_NONE, out)
    assert torch.allclose(out.cpu(), onr.rmsnorm(x, w), rtol=1e-5, atol=1e-6)


def test_cache_position_wraps_and_invalid_writes_nothing(dev):
    """A cache of cache_rows rows is a ring: position p lands at row p mod cache_rows (40 -> 8 of 32,
    the bounded window of oracle/v4_fast.py:93-96); a negative position, or one past the rotation
    table, writes nothing."""
    from smla import _lib, ops
    from smla import norm_rope as snr
    announce("row_epilogue cache ring positions")
    cos_d, sin_d = snr.rope_tables(64, 64, *YARN, device=dev)
    cache = torch.zeros(4, 32, 512, dtype=torch.bfloat16, device=dev)
    x = torch.ones(4, 512, device=dev)
    ops.row_epilogue(x, None, torch.tensor([5, 40, -1, 70], dtype=torch.int32, device=dev), cos_d, sin_d, 64,
                     _lib.SIM_FP8, cache, cache_rows=32)
    c = cache.float().cpu()
    assert c[0, 5].abs().sum() > 0 and c[1, 8].abs().sum() > 0
    c[0, 5] = 0
    c[1, 8] = 0
    assert c.abs().sum() == 0


@pytest.mark.parametrize("ratio,n_raw", [(4, 512), (0, 512), (4, 128), (0, 200)])
def test_decode_ids_brute_force(dev, ratio, n_raw):
    """Window ids: position pp at raw row pp mod n_raw (a cache with a row per position, or a ring
    of 128 or 200 rows that positions up to 511 wrap), then the visible compressed rows."""
    from smla import ops
    announce(f"decode_ids ratio={ratio} n_raw={n_raw}")
    ncomp, d, W = 128, 512, 128
    pos = torch.tensor([0, 3, 126, 127, 128, 300, 511], dtype=torch.int32)
    B = pos.numel()
    T = W + (ncomp if ratio else 0)
    comp32 = torch.randn(B, ncomp, d) if ratio else None
    comp_out = torch.zeros(B, ncomp, d, dtype=torch.bfloat16, device=dev) if ratio else None
    ids = ops.decode_ids(pos.to(dev), W, ratio, n_raw, ncomp, T, comp32=None if comp32 is None else comp32.to(dev),
                         comp_out=comp_out).cpu()
    for b in range(B):
        p = int(pos[b])
        lo = max(0, p - W + 1)
        win = [t % n_raw for t in range(lo, p + 1)] + [-1] * (W - (p + 1 - lo))
        comp = [n_raw + j for j in range(ncomp) if ratio and j < (p + 1) // ratio]
        comp += [-1] * (T - W - len(comp))
        assert ids[b].tolist() == win + comp
        if ratio:
            got = comp_out[b].cpu()
            r = (p + 1) // ratio - 1
            if (p + 1) % ratio == 0:
                assert torch.equal(got[r], comp32[b, r].to(torch.bfloat16))
                got[r] = 0
            assert torch.all(got.float() == 0)


def test_row_epilogue_ids_equals_separate_calls(dev):
    """smla_row_epilogue_ids (the per-head q epilogue and the decode id build in one launch) against
    smla_row_epilogue then smla_decode_ids on the same inputs: q rows, ids and the emitted
    compressed rows' bf16 copies bit for bit, with positions that emit, that do not, and one
    negative position."""
    from smla import _lib, ops
    announce("row epilogue + decode ids in one launch")
    g = torch.Generator().manual_seed(12)
    B, H, d, rd, n_pos, ncomp, n_raw, window = 4, 64, 512, 64, 4096, 300, 4096, 128
    T = window + ncomp
    x = torch.randn(B * H, d, generator=g).to(dev)
    cos_t = torch.randn(n_pos, rd // 2, generator=g).to(dev)
    sin_t = torch.randn(n_pos, rd // 2, generator=g).to(dev)
    comp32 = torch.randn(B, ncomp, d, generator=g).to(dev)
    pos = torch.tensor([3, 1000, -1, 1199], dtype=torch.int32, device=dev)   # 3, 1199: a row completes
    outs = []
    for fused in (False, True):
        q = torch.zeros(B, H, d, dtype=torch.bfloat16, device=dev)
        ids = torch.zeros(B, T, dtype=torch.int32, device=dev)
        comp_out = torch.zeros(B, ncomp, d, dtype=torch.bfloat16, device=dev)
        if fused:
            ops.row_epilogue_ids(x, None, pos, cos_t, sin_t, rd, _lib.SIM_NONE, q, H, pos, window, 4, n_raw, ncomp, T,
                                 ids, comp32=comp32, comp_out=comp_out)
        else:
            ops.row_epilogue(x, None, pos, cos_t, sin_t, rd, _lib.SIM_NONE, q, rows_per_pos=H)
            ops.decode_ids(pos, window, 4, n_raw, ncomp, T, out=ids, comp32=comp32, comp_out=comp_out)
        outs.append((q, ids, comp_out))
    torch.cuda.synchronize()
    (q0, i0, c0), (q1, i1, c1) = outs
    assert torch.equal(q0.view(torch.int16), q1.view(torch.int16))
    assert torch.equal(i0, i1)
    assert torch.equal(c0.view(torch.int16), c1.view(torch.int16))
    assert q0.float().abs().sum() > 0 and c0.float().abs().sum() > 0 and (i0 >= 0).any()
