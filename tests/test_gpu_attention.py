"""GPU parity of smla_sparse_attn against the CPU oracle (ref_torch/sparse_attn.py semantics).

Tolerances: fp32 path 1e-5 max-abs; bf16 path max-abs <= 2e-2, max-abs / max|ref| <= 1e-2, and per
element |out - ref| <= 1e-2 |ref| + 4e-3 max|ref| (the oracle runs in fp32 on the exact bf16 /
dequantised-fp8 input values)."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import sparse_attn as osa

pytestmark = pytest.mark.gpu

BF16_ABS, BF16_REL, F32_ABS = 2e-2, 1e-2, 1e-5


def _check_bf16(out, ref, what):
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


def _oracle_two_source(q, kv0, kv1, sink, idx, scale, dv):
    """q [B,S,H,D], kv0 [B,n0,D], kv1 [B,n1,D] or None, idx [B,S,T]; out-of-range ids masked."""
    outs = []
    for b in range(q.shape[0]):
        kv = kv0[b].float() if kv1 is None else torch.cat([kv0[b].float(), kv1[b].float()])
        ib = idx[b].long().clone()
        ib[(ib < 0) | (ib >= kv.shape[0])] = -1
        outs.append(osa.sparse_attn(q[b].float(), kv, sink, ib, scale, dv=dv))
    return torch.stack(outs)


def _lib():
    from smla import _lib
    return _lib.lib()


def test_fp32_generic_path_small(dev):
    from smla import sparse_attn as ssa
    g = torch.Generator().manual_seed(0)
    # D 576 / 40 / 64: rows held in registers; 700: 16 register chunks; 1100: the dot in blocks of
    # 16 chunks, value columns loaded again
    for (s, h, d, n, T, dv) in [(1, 16, 576, 300, 100, 512), (3, 5, 40, 50, 33, 40), (2, 2, 64, 10, 300, 32),
                                (2, 3, 700, 400, 150, 512), (1, 4, 1100, 300, 77, 700)]:
        announce(f"fp32 generic s={s} h={h} d={d} n={n} T={T}")
        q = torch.randn(s, h, d, generator=g)
        kv = torch.randn(n, d, generator=g)
        idx = torch.randint(-1, n, (s, T), generator=g, dtype=torch.int32)
        sink = torch.randn(h, generator=g)
        out = ssa.sparse_attn(q.to(dev), kv.to(dev), sink.to(dev), idx.to(dev), d ** -0.5, dv=dv)
        ref = osa.sparse_attn(q, kv, sink, idx, d ** -0.5, dv=dv)
        assert (out.cpu() - ref).abs().max().item() <= F32_ABS


@pytest.mark.parametrize("B,S,H,T,n0,n1,use_sink,D,sharp", [
    (1, 1, 64, 32, 100, 0, False, 576, 1.0),
    (1, 1, 64, 33, 100, 0, True, 576, 1.0),
    (2, 1, 64, 2176, 4000, 1000, False, 576, 1.0),
    (2, 3, 64, 300, 500, 300, True, 576, 50.0),
    (1, 2, 16, 70, 200, 0, True, 576, 20.0),
    (1, 1, 128, 257, 300, 40, False, 576, 1.0),
    (3, 1, 32, 96, 256, 0, True, 512, 10.0),
    (1, 1, 48, 1000, 3000, 0, False, 576, 30.0),
])
def test_bf16_mfma_vs_oracle(dev, B, S, H, T, n0, n1, use_sink, D, sharp):
    from smla import sparse_attn as ssa
    announce(f"bf16 mfma B={B} S={S} H={H} T={T} n0={n0} n1={n1} D={D} sharp={sharp}")
    g = torch.Generator().manual_seed(B * 1000 + T)
    q = (torch.randn(B, S, H, D, generator=g) * 0.05 * sharp).to(torch.bfloat16)
    kv0 = (torch.randn(B, n0, D, generator=g) * 0.5).to(torch.bfloat16)
    kv1 = (torch.randn(B, n1, D, generator=g) * 0.5).to(torch.bfloat16) if n1 else None
    idx = torch.randint(0, n0 + n1, (B, S, T), generator=g, dtype=torch.int32)
    # -1 padding, a duplicate and an out-of-range id
    idx[..., -min(5, T - 1):] = -1
    if T > 3:
        idx[..., 1] = idx[..., 0]
        idx[..., 2] = n0 + n1 + 7
    sink = torch.randn(H, generator=g) if use_sink else None
    scale = D ** -0.5
    out = ssa.sparse_attn_two_source(q.to(dev), kv0.to(dev), None if kv1 is None else kv1.to(dev),
                                     None if sink is None else sink.to(dev), idx.to(dev), scale, dv=512)
    ref = _oracle_two_source(q, kv0, kv1, sink, idx, scale, 512)
    _check_bf16(out, ref, "bf16 mfma")


def test_bf16_split_plans_agree(dev):
    """Every split count (1 = direct epilogue, many = LSE merge) gives the oracle's answer."""
    from smla import ops
    g = torch.Generator().manual_seed(7)
    B, H, D, n, T = 2, 64, 576, 3000, 1500
    q = (torch.randn(B, 1, H, D, generator=g) * 0.5).to(torch.bfloat16)
    kv = (torch.randn(B, n, D, generator=g) * 0.5).to(torch.bfloat16)
    idx = torch.randint(0, n, (B, 1, T), generator=g, dtype=torch.int32)
    ref = _oracle_two_source(q, kv, None, None, idx, D ** -0.5, 512)
    qd, kvd, idxd = q.to(dev), kv.to(dev), idx.to(dev)
    seen = set()
    for rps in (0, 32, 64, 96, 320, 1504, 8192):
        ns, got_rps, _ = ops.attn_plan(B, 1, H, D, 512, T, rows_per_split=rps)
        announce(f"split plan rows_per_split={rps} -> nsplit={ns} rows={got_rps}")
        seen.add(ns)
        out = ops.sparse_attn_ex(qd, kvd, None, None, None, None, idxd, D ** -0.5, 512, rows_per_split=rps)
        _check_bf16(out, ref, f"rows_per_split {rps}")
    assert 1 in seen and max(seen) >= 40, seen


def test_many_splits_merge(dev):
    """141 splits of 32 rows per query row (more than one load chunk and more splits than merge
    threads), 16 sequences, a sink and scattered -1 ids: the merge gives the oracle's answer."""
    from smla import sparse_attn as ssa
    g = torch.Generator().manual_seed(11)
    B, H, D, n, T = 16, 64, 576, 5000, 4500
    announce(f"many splits B={B} T={T}")
    q = (torch.randn(B, 1, H, D, generator=g) * 0.3).to(torch.bfloat16)
    kv = (torch.randn(B, n, D, generator=g) * 0.5).to(torch.bfloat16)
    idx = torch.randint(0, n, (B, 1, T), generator=g, dtype=torch.int32)
    idx[:, :, ::7] = -1
    sink = torch.randn(H, generator=g)
    ref = _oracle_two_source(q, kv, None, sink, idx, D ** -0.5, 512)
    from smla import ops
    ns, _, _ = ops.attn_plan(B, 1, H, D, 512, T, rows_per_split=32)
    assert ns > 128, ns
    out = ops.sparse_attn_ex(q.to(dev), kv.to(dev), None, None, None, sink.to(dev), idx.to(dev), D ** -0.5, 512,
                             rows_per_split=32)
    _check_bf16(out, ref, "many splits")


@pytest.mark.parametrize("nsplit", [2, 8, 9, 16, 17, 24, 25, 32, 33, 48, 64, 65, 97, 128, 129])
def test_merge_split_counts(dev, nsplit):
    """Split counts on both sides of the merge's chunk sizes (8, 16, 24 and 32 splits per load
    chunk) and wave counts (one wave per piece up to 32 splits, two up to 64, four beyond, several
    chunks per wave past 128): 32-row splits of bf16 rows, a sink, two 64-head groups, bf16
    partials in fragment order, against the oracle."""
    from smla import ops
    g = torch.Generator().manual_seed(100 + nsplit)
    B, H, D, n = 2, 128, 576, 3000
    T = 32 * nsplit - 5
    announce(f"merge nsplit={nsplit} T={T} H={H}")
    q = (torch.randn(B, 1, H, D, generator=g) * 0.3).to(torch.bfloat16)
    kv = (torch.randn(B, n, D, generator=g) * 0.5).to(torch.bfloat16)
    idx = torch.randint(0, n, (B, 1, T), generator=g, dtype=torch.int32)
    sink = torch.randn(H, generator=g)
    ns, rps, _ = ops.attn_plan(B, 1, H, D, 512, T, rows_per_split=32)
    assert ns == nsplit and rps == 32, (ns, rps)
    out = ops.sparse_attn_ex(q.to(dev), kv.to(dev), None, None, None, sink.to(dev), idx.to(dev), D ** -0.5, 512,
                             rows_per_split=32)
    _check_bf16(out, _oracle_two_source(q, kv, None, sink, idx, D ** -0.5, 512), f"merge of {nsplit} splits")


def test_all_masked_rows_are_nan(dev):
    from smla import sparse_attn as ssa
    announce("all-masked rows")
    g = torch.Generator().manual_seed(9)
    q = (torch.randn(2, 2, 64, 576, generator=g) * 0.1).to(torch.bfloat16)
    kv = (torch.randn(2, 64, 576, generator=g)).to(torch.bfloat16)
    idx = torch.randint(0, 64, (2, 2, 40), generator=g, dtype=torch.int32)
    idx[0, 1] = -1
    out = ssa.sparse_attn_batched(q.to(dev), kv.to(dev), torch.zeros(64, device=dev), idx.to(dev), 0.04, dv=512).cpu()
    assert torch.isnan(out[0, 1].float()).all()
    assert not torch.isnan(out[0, 0].float()).any() and not torch.isnan(out[1].float()).any()
    # fp32 generic path too
    out32 = ssa.sparse_attn(q[0].float().to(dev), kv[0].float().to(dev), None, idx[0].to(dev), 0.04, dv=512).cpu()
    assert torch.isnan(out32[1]).all() and not torch.isnan(out32[0]).any()


@pytest.mark.parametrize("S,H,T,masked", [(1, 1, 4000, "none"), (2, 4, 300, "first"), (1, 3, 200, "all"),
                                           (1, 16, 512, "scattered")])
def test_generic_split_states(dev, S, H, T, masked):
    """The vector-ALU kernel over list splits (up to 64: about one workgroup per compute unit for
    few (row, head) pairs) and its merge: fp32 rows against the oracle at 1e-5 with a sink, splits
    whose entries are all masked (weight zero), rows with no valid entry (NaN), and the split and
    merge phases run as separate calls equal, bit for bit, to the call that runs both."""
    from smla import _lib, ops
    g = torch.Generator().manual_seed(T + H)
    D, dv, n = 576, 512, 900
    announce(f"generic split states S={S} H={H} T={T} masked={masked}")
    q = torch.randn(1, S, H, D, generator=g)
    kv = torch.randn(1, n, D, generator=g)
    idx = torch.randint(0, n, (1, S, T), generator=g, dtype=torch.int32)
    if masked == "first":
        idx[..., : T // 2] = -1        # the first splits see no valid entry
    elif masked == "all":
        idx[...] = -1
    elif masked == "scattered":
        idx[..., ::3] = -1
    sink = torch.randn(H, generator=g)
    scale = D ** -0.5
    ns, _, wsb = ops.attn_plan(1, S, H, D, dv, T, torch.float32, torch.float32, torch.float32)
    assert ns == 0 and wsb > 0  # the vector-ALU kernel, with split states in the workspace
    qd, kvd, idxd, sinkd = q.to(dev), kv.to(dev), idx.to(dev), sink.to(dev)
    out = ops.sparse_attn_ex(qd, kvd, None, None, None, sinkd, idxd, scale, dv)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    o2 = torch.empty_like(out)
    ops.sparse_attn_ex(qd, kvd, None, None, None, sinkd, idxd, scale, dv, phases=_lib.ATTN_SPLIT, out=o2, workspace=ws)
    ops.sparse_attn_ex(qd, kvd, None, None, None, sinkd, idxd, scale, dv, phases=_lib.ATTN_MERGE, out=o2, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(out, o2) or (torch.isnan(out).all() and torch.isnan(o2).all())
    out = out.cpu()[0]
    if masked == "all":
        assert torch.isnan(out).all()
        return
    ref = osa.sparse_attn(q[0], kv[0], sink, idx[0], scale, dv=dv)
    assert (out - ref).abs().max().item() <= F32_ABS


@pytest.mark.parametrize("B,T,n,sharp,H,D,pow2", [(1, 64, 200, 1.0, 64, 576, True), (3, 700, 2000, 40.0, 64, 576, True),
                                                (2, 2048, 2048, 1.0, 64, 576, True), (2, 333, 900, 10.0, 48, 576, True),
                                                (2, 300, 500, 5.0, 64, 512, True), (2, 700, 1500, 10.0, 64, 576, False)])
def test_fp8_rows_vs_oracle(dev, B, T, n, sharp, H, D, pow2):
    """e4m3 rows with per-64 fp32 scales: powers of two (the fp8 simulation's form) and, with
    pow2=False, amax/448 (any fp32 scale: row value = decode(code) * scale)."""
    from smla import sparse_attn as ssa
    from smla import workloads as wl
    announce(f"fp8 rows B={B} T={T} n={n} H={H} D={D} pow2={pow2}")
    g = torch.Generator().manual_seed(T)
    q = (torch.randn(B, 1, H, D, generator=g) * 0.05 * sharp).to(torch.bfloat16)
    x = torch.randn(B, n, D, generator=g) * 0.05
    if pow2:
        codes, scales = wl.quant_e4m3_pow2(x)
    else:
        blk = x.reshape(B, n, D // 64, 64)
        scales = blk.abs().amax(-1).clamp_min(1e-4) / 448.0
        codes = (blk / scales[..., None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).reshape(B, n, D)
        assert (scales.view(torch.int32) & 0x7FFFFF).ne(0).float().mean() > 0.9  # not powers of two
    idx = torch.randint(0, n, (B, 1, T), generator=g, dtype=torch.int32)
    idx[..., :3] = -1
    idx[..., -2:] = -1
    out = ssa.sparse_attn_batched(q.to(dev), codes.to(dev), None, idx.to(dev), D ** -0.5, dv=512,
                                  kv_scale=scales.to(dev))
    rows = wl.dequant_e4m3(codes, scales)
    ref = _oracle_two_source(q, rows, None, None, idx, D ** -0.5, 512)
    _check_bf16(out, ref, "fp8 rows")



@pytest.mark.parametrize("D", [576, 512])
def test_fp8_split_plans_and_fp32_out(dev, D):
    """fp8 rows under every kind of split plan (splits of up to 256 rows: the 4-slot ring, longer:
    the 3-slot ring with the long index table), with bf16 and fp32 outputs (one split: the
    kernel's own epilogue, whose fp32 rows are staged in LDS past the tile loop's data; more: the
    merge of bf16 or fp32 partial states): every combination gives the oracle's answer."""
    from smla import ops
    from smla import workloads as wl
    g = torch.Generator().manual_seed(D)
    B, H, n, T = 2, 64, 3000, 1500
    q = (torch.randn(B, 1, H, D, generator=g) * 0.3).to(torch.bfloat16)
    codes, scales = wl.quant_e4m3_pow2(torch.randn(B, n, D, generator=g) * 0.05)
    idx = torch.randint(0, n, (B, 1, T), generator=g, dtype=torch.int32)
    idx[..., ::11] = -1
    ref = _oracle_two_source(q, wl.dequant_e4m3(codes, scales), None, None, idx, D ** -0.5, 512)
    qd, cd, sd, idxd = q.to(dev), codes.to(dev), scales.to(dev), idx.to(dev)
    for rps in (32, 96, 512, 544, 1504):
        ns, got_rps, _ = ops.attn_plan(B, 1, H, D, 512, T, torch.bfloat16, torch.uint8, rows_per_split=rps)
        for odt in (torch.bfloat16, torch.float32):
            announce(f"fp8 D={D} rows_per_split={rps} (nsplit {ns}) out {odt}")
            out = torch.empty(B, 1, H, 512, dtype=odt, device=dev)
            ops.sparse_attn_ex(qd, cd, None, sd, None, None, idxd, D ** -0.5, 512, rows_per_split=rps, out=out)
            _check_bf16(out, ref, f"fp8 rows_per_split {rps} out {odt}")


@pytest.mark.parametrize("kind,S,H,D,dv,T,n", [("bf16", 3, 8, 128, 128, 300, 500),      # H % 16 != 0
                                               ("bf16", 2, 16, 256, 200, 90, 400),      # D, DV off the MFMA shapes
                                               ("fp8", 2, 8, 128, 128, 257, 600),       # fp8 rows, H = 8
                                               ("fp8", 1, 20, 192, 64, 70, 300)])
def test_generic_kernel_bf16_fp8_rows(dev, kind, S, H, D, dv, T, n):
    """Shapes the MFMA split kernel does not take (H not a multiple of 16, D other than 576 / 512,
    DV other than 512) run the vector-ALU kernel for bf16 and fp8 rows as well as fp32: the same
    results as the oracle on the exact bf16 / dequantised fp8 values, to the bf16 tolerance."""
    from smla import sparse_attn as ssa
    from smla import workloads as wl
    announce(f"generic kernel {kind} S={S} H={H} D={D} dv={dv} T={T} n={n}")
    g = torch.Generator().manual_seed(S * 100 + H)
    B = 2
    q = (torch.randn(B, S, H, D, generator=g) * 0.3).to(torch.bfloat16)
    x = torch.randn(B, n, D, generator=g) * 0.3
    idx = torch.randint(-1, n, (B, S, T), generator=g, dtype=torch.int32)
    sink = torch.randn(H, generator=g)
    if kind == "bf16":
        kv = x.to(torch.bfloat16)
        out = ssa.sparse_attn_batched(q.to(dev), kv.to(dev), sink.to(dev), idx.to(dev), D ** -0.5, dv=dv)
        rows = kv.float()
    else:
        codes, scales = wl.quant_e4m3_pow2(x)
        out = ssa.sparse_attn_batched(q.to(dev), codes.to(dev), sink.to(dev), idx.to(dev), D ** -0.5, dv=dv,
                                      kv_scale=scales.to(dev))
        rows = wl.dequant_e4m3(codes, scales)
    ref = _oracle_two_source(q, rows, None, sink, idx, D ** -0.5, dv)
    _check_bf16(out, ref, f"generic kernel {kind}")


def test_fp32_plumbing_workload(dev):
    """The fp32 plumbing case: H=16, 4096 rows, indexer top-512, fp32 attention, 1e-5."""
    from smla import indexer as sidx
    from smla import sparse_attn as ssa
    from smla import workloads as wl
    from oracle import indexer as oidx
    announce("fp32 plumbing workload")
    w = wl.fp32_plumbing()
    sc = sidx.indexer_score(w["q_idx"][None].to(dev), w["k_idx"][None].to(dev), None, w["w"][None].to(dev))
    sc_ref = oidx.indexer_score(w["q_idx"].numpy(), w["k_idx"].numpy(), None, w["w"].numpy())
    np.testing.assert_array_equal(sc[0].cpu().numpy().view(np.uint32), sc_ref.view(np.uint32))
    sel = sidx.topk(sc[0], w["k"])
    sel_ref = oidx.topk(sc_ref, w["k"])
    np.testing.assert_array_equal(sel.cpu().numpy(), sel_ref)
    out = ssa.sparse_attn(w["q"].to(dev), w["kv"].to(dev), None, sel, w["scale"], dv=w["dv"])
    ref = osa.sparse_attn(w["q"], w["kv"], None, torch.from_numpy(sel_ref), w["scale"], dv=w["dv"])
    assert (out.cpu() - ref).abs().max().item() <= F32_ABS


def test_decode_32k_full_size(dev):
    """Full 32K decode step (B=8): indexer scores bit-exact, selected sets exact, attention
    within bf16 tolerance."""
    from smla import indexer as sidx
    from smla import sparse_attn as ssa
    from smla import workloads as wl
    from smla import compressor as scomp
    from oracle import indexer as oidx
    from oracle import compressor as ocomp
    announce("decode_32k full size")
    w = wl.decode_32k()
    B, k, win, n_raw = 8, w["k"], w["window"], w["raw"].shape[1]
    raw = w["raw"].to(dev)
    comp = scomp.block_mean_pool(raw, 4)
    comp_ref = ocomp.mean_pool(w["raw"], 4).to(torch.bfloat16)
    assert torch.equal(comp.cpu(), comp_ref)
    pos = torch.full((B,), w["pos"], dtype=torch.int32, device=dev)
    sc = sidx.indexer_score(w["q_idx"].to(dev), w["k_codes"].to(dev), w["kscale"].to(dev), w["w"].to(dev))
    idx = sidx.select_decode_indices(sc[:, 0], k, pos, win, n_raw)
    out = ssa.sparse_attn_two_source(w["q"].to(dev), raw, comp, None, idx[:, None, :], w["scale"], dv=512)
    from smla.workloads import dequant_e4m3
    keys = dequant_e4m3(w["k_codes"], w["kscale"][..., None], block=64)
    sc_cpu = sc.cpu().numpy()
    for b in range(B):
        sref = oidx.indexer_score(w["q_idx"][b].float().numpy(), keys[b].numpy(), None, w["w"][b].numpy())
        # kscale applied last: recompute with the scale to keep the exact chain
        sref = oidx.indexer_score(w["q_idx"][b].float().numpy(),
                                  w["k_codes"][b].view(torch.float8_e4m3fn).float().numpy(),
                                  w["kscale"][b].numpy(), w["w"][b].numpy())
        np.testing.assert_array_equal(sc_cpu[b].view(np.uint32), sref.view(np.uint32))
        sel_ref = oidx.topk(sref, k)[0]
        ids_ref = np.concatenate([np.arange(w["pos"] - win + 1, w["pos"] + 1), sel_ref + n_raw]).astype(np.int32)
        np.testing.assert_array_equal(idx[b].cpu().numpy(), ids_ref)
    ref = _oracle_two_source(w["q"], w["raw"], comp_ref, None, idx[:, None, :].cpu(), w["scale"], 512)
    _check_bf16(out, ref, "decode_32k")


def test_batched_fp8_full_size(dev):
    from smla import sparse_attn as ssa
    from smla import workloads as wl
    announce("batched_fp8 full size")
    w = wl.batched_fp8()
    out = ssa.sparse_attn_batched(w["q"].to(dev), w["codes"].to(dev), None, w["idx"].to(dev), w["scale"],
                                  dv=512, kv_scale=w["scales"].to(dev))
    assert out.dtype == torch.bfloat16 and out.shape == (64, 1, 64, 512)
    outs = out.float().cpu()
    for b in range(64):
        rows = wl.dequant_e4m3(w["codes"][b], w["scales"][b])
        ref = osa.sparse_attn(w["q"][b].float(), rows, None, w["idx"][b].long(), w["scale"], dv=512)
        _check_bf16(outs[b], ref, f"batched_fp8 b={b}")
