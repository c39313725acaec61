"""GPU parity of the prefill form of smla_sparse_attn: S queries of one sequence, each attending
its 128-row raw window and every causally visible block-4 compressed row (the engine's index
build, oracle/decode_engine.py:110-114, at positions q_pos0..q_pos0+S-1), H=64, 576-wide bf16
rows, one split per query (long index lists; -1 padding at the end is trimmed by the kernel).

Tolerance: bf16 path, max-abs <= 2e-2 and max-abs / max|ref| <= 1e-2 against the fp32 oracle on
the same bf16 inputs."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import sparse_attn as osa

pytestmark = pytest.mark.gpu

BF16_ABS, BF16_REL = 2e-2, 1e-2


def _check(out, ref, what):
    out = out.float().cpu()
    assert not torch.isnan(out).any(), what
    err = (out - ref).abs().max().item()
    rel = err / max(ref.abs().max().item(), 1e-30)
    assert err <= BF16_ABS and rel <= BF16_REL, f"{what}: max abs {err:.3e}, rel {rel:.3e}"
    # element-wise as well: |out - ref| <= BF16_REL |ref| + 4e-3 max|ref| for every element.  The
    # floor covers the bf16 rounding of the softmax weights (2^-9 relative each): it bounds an
    # element's error by about 2^-9 of the values it averages, not of its own (possibly
    # cancelling) value; the largest seen is 2.6e-3 max|ref|
    bound = BF16_REL * ref.abs() + 4e-3 * ref.abs().max()
    bad = ((out - ref).abs() > bound).sum().item()
    worst = (((out - ref).abs() - BF16_REL * ref.abs()) / ref.abs().max()).max().item()
    assert bad == 0, f"{what}: {bad} elements outside rel {BF16_REL} + 4e-3 max|ref| (worst floor {worst:.2e})"


def _inputs(n_raw, S, H, seed, sharp=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(1, S, H, 576, generator=g) * 0.05 * sharp).to(torch.bfloat16)
    raw = (torch.randn(1, n_raw, 576, generator=g) * 0.5).to(torch.bfloat16)
    return q, raw


@pytest.mark.parametrize("one_split", [False, True], ids=["split_plan", "one_split_per_query"])
@pytest.mark.parametrize("n_raw,q_pos0,S,H,use_sink", [
    (4096, 4096 - 48, 48, 64, False),   # full lists: 128 window + 1024 compressed rows
    (4096, 0, 40, 64, True),            # first positions: short lists, mostly -1 padding
    (1024, 500, 33, 32, False),         # partial head group, mid-sequence
    (1024, 0, 1024, 64, True),          # 1024 query rows: the XCD-chunked row order, every row checked
])
def test_prefill_vs_oracle(dev, n_raw, q_pos0, S, H, use_sink, one_split):
    """one_split forces the single-split plan (3-tile ring, long index table) that the full
    4096-query prefill uses; otherwise these small query counts get short splits and a merge."""
    from smla import compressor as scomp
    from smla import ops
    from smla import workloads as wl
    announce(f"prefill n_raw={n_raw} q_pos0={q_pos0} S={S} H={H} sink={use_sink} one_split={one_split}")
    q, raw = _inputs(n_raw, S, H, seed=q_pos0 + S)
    raw_d = raw.to(dev)
    comp_d = scomp.block_mean_pool(raw_d, 4)
    comp = comp_d.cpu()
    # ids for the S query positions (the lists are built for all n_raw positions, rows taken)
    idx_all = wl.prefill_indices(n_raw, ratio=4, window=128, n_raw=n_raw)
    idx = idx_all[q_pos0:q_pos0 + S]
    sink = torch.randn(H, generator=torch.Generator().manual_seed(5)) if use_sink else None
    scale = 576 ** -0.5
    T = idx.shape[-1]
    rps = (T + 31) // 32 * 32 if one_split else 0
    out = ops.sparse_attn_ex(q.to(dev), raw_d, comp_d, None, None, None if sink is None else sink.to(dev),
                             idx[None].to(dev), scale, 512, rows_per_split=rps)
    if one_split:
        assert ops.attn_plan(1, S, H, 576, 512, T, rows_per_split=rps)[0] == 1
    torch.cuda.synchronize()
    kv = torch.cat([raw[0].float(), comp[0].float()])
    ref = osa.sparse_attn(q[0].float(), kv, sink, idx, scale, dv=512)
    _check(out[0], ref, "prefill")


@pytest.mark.parametrize("n_raw,q_pos0,S,H,ratio,use_sink", [
    (4096, 4096 - 48, 48, 64, 4, False),  # full lists
    (4096, 0, 40, 64, 4, True),           # first positions: windows shorter than 128
    (1024, 500, 33, 32, 4, False),        # partial head group, mid-sequence
    (1024, 0, 1024, 64, 4, True),         # XCD-chunked, longest-first order over 1024 queries
    (600, 100, 200, 64, 0, False),        # a window-only layer (ratio 0)
    (2000, 1500, 64, 128, 4, True),       # two head groups
])
def test_prefill_attn_implicit_rows(dev, n_raw, q_pos0, S, H, ratio, use_sink):
    """smla_prefill_attn (row sets computed in the kernel) equals the single-split attention over
    the explicit prefill index lists bit for bit, and the oracle within the bf16 tolerance."""
    from smla import compressor as scomp
    from smla import ops
    from smla import sparse_attn as ssa
    from smla import workloads as wl
    announce(f"prefill_attn n_raw={n_raw} q_pos0={q_pos0} S={S} H={H} ratio={ratio} sink={use_sink}")
    q, raw = _inputs(n_raw, S, H, seed=q_pos0 + S + 7)
    raw_d = raw.to(dev)
    comp_d = scomp.block_mean_pool(raw_d, 4) if ratio else None
    sink = torch.randn(H, generator=torch.Generator().manual_seed(6)) if use_sink else None
    sink_d = None if sink is None else sink.to(dev)
    scale = 576 ** -0.5
    out = ssa.prefill_attn(q.to(dev), raw_d, comp_d, sink_d, scale, q_pos0=q_pos0, window=128, ratio=ratio)
    idx_all = wl.prefill_indices(n_raw, ratio=4, window=128, n_raw=n_raw)
    idx = (idx_all if ratio else idx_all[:, :128])[q_pos0:q_pos0 + S]
    T = idx.shape[-1]
    rps = (T + 31) // 32 * 32
    ref_gpu = ops.sparse_attn_ex(q.to(dev), raw_d, comp_d, None, None, sink_d, idx[None].to(dev), scale, 512,
                                 rows_per_split=rps)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref_gpu.view(torch.int16)), "implicit rows differ from the index lists"
    kv = raw[0].float() if not ratio else torch.cat([raw[0].float(), comp_d.cpu()[0].float()])
    ref = osa.sparse_attn(q[0].float(), kv, sink, idx, scale, dv=512)
    _check(out[0], ref, "prefill_attn")


def test_prefill_attn_fp32_out(dev):
    """fp32 output (64 head rows of 2048 bytes staged in LDS after the tile loop): the bf16
    output's values before their rounding, so rounding them to bf16 gives the bf16 output bit for
    bit, and every head (the last ones included) within tolerance of the oracle."""
    from smla import compressor as scomp
    from smla import sparse_attn as ssa
    from smla import workloads as wl
    n_raw, q_pos0, S, H = 1024, 900, 40, 64
    announce(f"prefill_attn fp32 out n_raw={n_raw} q_pos0={q_pos0} S={S}")
    q, raw = _inputs(n_raw, S, H, seed=31)
    raw_d = raw.to(dev)
    comp_d = scomp.block_mean_pool(raw_d, 4)
    sink = torch.randn(H, generator=torch.Generator().manual_seed(8))
    scale = 576 ** -0.5
    out16 = ssa.prefill_attn(q.to(dev), raw_d, comp_d, sink.to(dev), scale, q_pos0=q_pos0, window=128, ratio=4)
    out32 = ssa.prefill_attn(q.to(dev), raw_d, comp_d, sink.to(dev), scale, q_pos0=q_pos0, window=128, ratio=4,
                             out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert out32.dtype == torch.float32
    assert torch.equal(out32.to(torch.bfloat16).view(torch.int16), out16.view(torch.int16))
    idx = wl.prefill_indices(n_raw, ratio=4, window=128, n_raw=n_raw)[q_pos0:q_pos0 + S]
    kv = torch.cat([raw[0].float(), comp_d.cpu()[0].float()])
    ref = osa.sparse_attn(q[0].float(), kv, sink, idx, scale, dv=512)
    _check(out32[0], ref, "prefill_attn fp32 out")


def test_prefill_attn_long_lists(dev):
    """Lists past the 8192 rows an index table holds (positions near 40000: 128 window rows and up
    to 10000 compressed rows per query) against the oracle; the queries straddle the point where
    the compressed part stops growing (n_comp rows)."""
    from smla import compressor as scomp
    from smla import sparse_attn as ssa
    from smla import workloads as wl
    n_raw, q_pos0, S, H = 40000, 39990, 10, 16
    announce(f"prefill_attn long lists n_raw={n_raw} q_pos0={q_pos0} S={S} H={H}")
    q, raw = _inputs(n_raw, S, H, seed=11, sharp=4.0)
    raw_d = raw.to(dev)
    comp_d = scomp.block_mean_pool(raw_d, 4)[:, :9998]  # the last rows of the last queries cut off
    sink = torch.randn(H, generator=torch.Generator().manual_seed(8))
    scale = 576 ** -0.5
    out = ssa.prefill_attn(q.to(dev), raw_d, comp_d, sink.to(dev), scale, q_pos0=q_pos0, window=128, ratio=4)
    torch.cuda.synchronize()
    n_comp = comp_d.shape[1]
    idx = wl.prefill_indices(S, ratio=4, window=128, n_raw=n_raw, q_pos0=q_pos0)
    idx = idx[:, :128 + n_comp]
    idx = torch.where(idx >= n_raw + n_comp, torch.full_like(idx, -1), idx)
    kv = torch.cat([raw[0].float(), comp_d.cpu()[0].float()])
    ref = osa.sparse_attn(q[0].float(), kv, sink, idx, scale, dv=512)
    _check(out[0], ref, "prefill_attn long lists")


def test_prefill_attn_rejects(dev):
    """Positions past the raw rows are refused before any launch; lists longer than the 8192-row
    index table of the list path are taken (no table)."""
    from smla import _lib
    from smla import sparse_attn as ssa
    q = torch.zeros(1, 8, 64, 576, dtype=torch.bfloat16, device=dev)
    raw = torch.zeros(1, 100, 576, dtype=torch.bfloat16, device=dev)
    comp = torch.zeros(1, 25, 576, dtype=torch.bfloat16, device=dev)
    with pytest.raises(_lib.SmlaError):
        ssa.prefill_attn(q, raw, comp, None, 0.04, q_pos0=95)          # positions 95..102 > 99
    big_raw = torch.zeros(1, 40000, 576, dtype=torch.bfloat16, device=dev)
    big_comp = torch.zeros(1, 10000, 576, dtype=torch.bfloat16, device=dev)
    out = ssa.prefill_attn(q, big_raw, big_comp, None, 0.04, q_pos0=39000)  # lists of 128 + 9752 rows
    torch.cuda.synchronize()
    assert not torch.isnan(out).any() and float(out.float().abs().max()) == 0.0  # zero rows attend to zero


def test_prefill_4k_full_size(dev):
    """The full prefill workload (S=4096 queries over a 4096-row sequence): every query's output
    is computed on the GPU and checked against the oracle, and the empty-set guarantee holds (no
    NaN anywhere: every query sees itself)."""
    from smla import compressor as scomp
    from smla import sparse_attn as ssa
    from smla import workloads as wl
    announce("prefill_4k full size")
    w = wl.prefill_4k()
    q, raw = w["q"], w["raw"]
    raw_d = raw.to(dev)
    comp_d = scomp.block_mean_pool(raw_d, 4)
    idx = wl.prefill_indices(4096, ratio=4, window=128, n_raw=4096)
    out = ssa.sparse_attn_two_source(q.to(dev), raw_d, comp_d, None, idx[None].to(dev), w["scale"], dv=512)
    # the prefill entry with its row sets computed in the kernel: the same bits
    out_implicit = ssa.prefill_attn(q.to(dev), raw_d, comp_d, None, w["scale"], q_pos0=0, window=128, ratio=4)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out_implicit.view(torch.int16))
    assert not torch.isnan(out).any()
    kv = torch.cat([raw[0].float(), comp_d.cpu()[0].float()])
    outs = out[0].float().cpu()
    for q0 in range(0, 4096, 256):   # every query, 256 at a time (the oracle gathers [256, T, 576])
        ref = osa.sparse_attn(q[0, q0:q0 + 256].float(), kv, None, idx[q0:q0 + 256], w["scale"], dv=512)
        _check(outs[q0:q0 + 256], ref, f"prefill_4k queries {q0}..{q0 + 255}")
