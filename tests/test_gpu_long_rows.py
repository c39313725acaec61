"""GPU parity of attention calls with more query rows than one launch of the split kernel holds
(its grid takes at most 65528 query rows): the list path, the prompt path with row sets computed
in the kernel, and decode attention with the selection in the kernel run as launches over row
chunks -- whole sequences while one fits, else pieces of one sequence.

Every output row must equal, bit for bit, the same rows computed by calls of fewer rows (each one
launch), which checks every row of the chunked call; rows on both sides of the chunk boundaries
are also checked against the oracle within the bf16 tolerance of test_gpu_attention."""
import pytest
import torch

from conftest import announce
from test_gpu_attention import _check_bf16, _oracle_two_source

pytestmark = pytest.mark.gpu

CHUNK = 65528


def _bits(t):
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t


def _same(a, b, what):
    torch.cuda.synchronize()
    assert torch.equal(_bits(a), _bits(b)), what


def _rows_near(S, bounds):
    """query rows at both ends and on both sides of each chunk boundary"""
    rows = {0, 1, S - 2, S - 1}
    for c in bounds:
        rows.update(r for r in range(c - 3, c + 3) if 0 <= r < S)
    return torch.tensor(sorted(rows))


def test_list_path_pieces_of_one_sequence(dev):
    """One sequence of 66000 query rows (launches of 65528 + 472 rows), two row sources, a sink,
    32-row splits (two per row: split kernel and merge per chunk, each chunk's partial states in
    its own stretch of the workspace)."""
    from smla import ops
    B, S, H, D, n0, n1, T = 1, 66000, 16, 576, 300, 60, 64
    announce(f"long list path B={B} S={S} H={H} T={T} rows_per_split=32")
    g = torch.Generator(device=dev).manual_seed(1)
    q = (torch.randn(B, S, H, D, generator=g, device=dev) * 0.3).to(torch.bfloat16)
    kv0 = (torch.randn(B, n0, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    kv1 = (torch.randn(B, n1, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    idx = torch.randint(-1, n0 + n1, (B, S, T), generator=g, device=dev, dtype=torch.int32)
    sink = torch.randn(H, generator=g, device=dev)
    scale = D ** -0.5
    ns, rps, _ = ops.attn_plan(B, S, H, D, 512, T, rows_per_split=32)
    assert (ns, rps) == (2, 32)
    out = ops.sparse_attn_ex(q, kv0, kv1, None, None, sink, idx, scale, 512, rows_per_split=32)
    for lo, hi in ((0, 40000), (40000, S)):
        part = ops.sparse_attn_ex(q[:, lo:hi].contiguous(), kv0, kv1, None, None, sink, idx[:, lo:hi].contiguous(),
                                  scale, 512, rows_per_split=32)
        _same(out[:, lo:hi], part, f"rows {lo}..{hi} differ from a call of those rows")
    rows = _rows_near(S, [CHUNK])
    ref = _oracle_two_source(q[:, rows].cpu(), kv0.cpu(), kv1.cpu(), sink.cpu(), idx[:, rows].cpu(), scale, 512)
    _check_bf16(out[:, rows], ref, "long list path")


def test_list_path_whole_sequences_fp8(dev):
    """Three sequences of 30000 query rows (launches of two sequences, then one: row sources and
    scales offset per chunk), fp8 rows in both sources with per-64 scales."""
    from smla import ops
    from smla import workloads as wl
    B, S, H, D, n0, n1, T = 3, 30000, 16, 576, 256, 64, 64
    announce(f"long fp8 list path B={B} S={S} H={H} T={T}")
    gc = torch.Generator().manual_seed(2)
    c0, s0 = wl.quant_e4m3_pow2(torch.randn(B, n0, D, generator=gc) * 0.05)
    c1, s1 = wl.quant_e4m3_pow2(torch.randn(B, n1, D, generator=gc) * 0.05)
    g = torch.Generator(device=dev).manual_seed(2)
    q = (torch.randn(B, S, H, D, generator=g, device=dev) * 0.3).to(torch.bfloat16)
    idx = torch.randint(-1, n0 + n1, (B, S, T), generator=g, device=dev, dtype=torch.int32)
    scale = D ** -0.5
    c0d, s0d, c1d, s1d = c0.to(dev), s0.to(dev), c1.to(dev), s1.to(dev)
    out = ops.sparse_attn_ex(q, c0d, c1d, s0d, s1d, None, idx, scale, 512, rows_per_split=64)
    for b in range(B):
        part = ops.sparse_attn_ex(q[b:b + 1].contiguous(), c0d[b:b + 1].contiguous(), c1d[b:b + 1].contiguous(),
                                  s0d[b:b + 1].contiguous(), s1d[b:b + 1].contiguous(), None,
                                  idx[b:b + 1].contiguous(), scale, 512, rows_per_split=64)
        _same(out[b:b + 1], part, f"sequence {b} differs from a call of that sequence")
    rows = _rows_near(S, [])
    for b in (1, 2):
        ref = _oracle_two_source(q[b:b + 1, rows].cpu(), wl.dequant_e4m3(c0[b:b + 1], s0[b:b + 1]),
                                 wl.dequant_e4m3(c1[b:b + 1], s1[b:b + 1]), None, idx[b:b + 1, rows].cpu(), scale, 512)
        _check_bf16(out[b:b + 1, rows], ref, f"long fp8 list path, sequence {b}")


def test_prefill_pieces_of_one_sequence(dev):
    """Prompt attention over 66000 positions of one sequence (launches of 65528 + 472 queries,
    the second starting at position 65528), window 128 and a 512-block compressed part."""
    from smla import sparse_attn as ssa
    from smla import workloads as wl
    S, H, D, ratio, window = 66000, 16, 576, 512, 128
    n_comp = S // ratio
    announce(f"long prefill S={S} H={H} ratio={ratio}")
    g = torch.Generator(device=dev).manual_seed(3)
    q = (torch.randn(1, S, H, D, generator=g, device=dev) * 0.3).to(torch.bfloat16)
    raw = (torch.randn(1, S, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    comp = (torch.randn(1, n_comp, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    sink = torch.randn(H, generator=g, device=dev)
    scale = D ** -0.5
    out = ssa.prefill_attn(q, raw, comp, sink, scale, q_pos0=0, window=window, ratio=ratio)
    for lo, hi in ((0, 40000), (40000, S)):
        part = ssa.prefill_attn(q[:, lo:hi].contiguous(), raw, comp, sink, scale, q_pos0=lo, window=window,
                                ratio=ratio)
        _same(out[:, lo:hi], part, f"positions {lo}..{hi} differ from a call of those positions")
    rows = _rows_near(S, [CHUNK])
    idx = wl.prefill_indices(S, ratio=ratio, window=window, n_raw=S)[rows]
    ref = _oracle_two_source(q[:, rows].cpu(), raw.cpu(), comp.cpu(), sink.cpu(), idx[None], scale, 512)
    _check_bf16(out[:, rows], ref, "long prefill")


def test_prefill_whole_sequences(dev):
    """Two sequences of 40000 positions (one launch each: raw rows offset per sequence), a
    window-only layer."""
    from smla import sparse_attn as ssa
    from smla import workloads as wl
    B, S, H, D, window = 2, 40000, 16, 576, 128
    announce(f"long prefill B={B} S={S} H={H} window only")
    g = torch.Generator(device=dev).manual_seed(4)
    q = (torch.randn(B, S, H, D, generator=g, device=dev) * 0.3).to(torch.bfloat16)
    raw = (torch.randn(B, S, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    scale = D ** -0.5
    out = ssa.prefill_attn(q, raw, None, None, scale, q_pos0=0, window=window, ratio=0)
    for b in range(B):
        part = ssa.prefill_attn(q[b:b + 1].contiguous(), raw[b:b + 1].contiguous(), None, None, scale, q_pos0=0,
                                window=window, ratio=0)
        _same(out[b:b + 1], part, f"sequence {b} differs from a call of that sequence")
    rows = _rows_near(S, [])
    idx = wl.prefill_indices(S, ratio=S + 1, window=window, n_raw=S)[rows]   # window entries only
    ref = _oracle_two_source(q[1:2, rows].cpu(), raw[1:2].cpu(), None, None, idx[None], scale, 512)
    _check_bf16(out[1:2, rows], ref, "long prefill, sequence 1")


def test_decode_attn_pieces_of_one_sequence(dev):
    """Decode attention with the selection in the attention workgroups over 66000 query rows of
    one sequence (launches of 65528 + 472 rows, scores / nvis / pos offset per chunk): equal to the
    selection followed by the list path, to calls of fewer rows, and to the oracle."""
    from smla import indexer as sidx
    from smla import sparse_attn as ssa
    B, S, H, D, n_raw, n_comp, N, k, window = 1, 66000, 16, 576, 256, 512, 512, 64, 128
    announce(f"long decode_attn S={S} H={H} N={N} k={k}")
    g = torch.Generator(device=dev).manual_seed(5)
    q = (torch.randn(B, S, H, D, generator=g, device=dev) * 0.3).to(torch.bfloat16)
    raw = (torch.randn(B, n_raw, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    comp = (torch.randn(B, n_comp, D, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    sc = torch.randn(B * S, N, generator=g, device=dev)
    pos = torch.randint(0, 5000, (B * S,), generator=g, device=dev, dtype=torch.int32)
    nvis = torch.randint(1, N + 1, (B * S,), generator=g, device=dev, dtype=torch.int32)
    sink = torch.randn(H, generator=g, device=dev)
    scale = D ** -0.5
    out = ssa.decode_attn(q, raw, comp, sink, sc, pos, window, k, scale, dv=512, nvis=nvis)
    idx = sidx.select_decode_indices(sc, k, pos, window, n_raw, nvis=nvis).view(B, S, -1)
    two = ssa.sparse_attn_two_source(q, raw, comp, sink, idx, scale, dv=512)
    _same(out, two, "differs from the selection followed by the list path")
    for lo, hi in ((0, 40000), (40000, S)):
        part = ssa.decode_attn(q[:, lo:hi].contiguous(), raw, comp, sink, sc[lo:hi].contiguous(),
                               pos[lo:hi].contiguous(), window, k, scale, dv=512, nvis=nvis[lo:hi].contiguous())
        _same(out[:, lo:hi], part, f"rows {lo}..{hi} differ from a call of those rows")
    rows = _rows_near(S, [CHUNK])
    ref = _oracle_two_source(q[:, rows].cpu(), raw.cpu(), comp.cpu(), sink.cpu(), idx[:, rows].cpu(), scale, 512)
    _check_bf16(out[:, rows], ref, "long decode_attn")


def _f32_bits(t):
    return t.contiguous().view(torch.int32)


def test_indexer_pieces_of_one_sequence(dev):
    """Indexer scores for 66000 query rows of one sequence (64 heads x 64 dims: the matrix-core
    kernel; launches of 65528 + 472 rows), fp8 keys with scales, ragged nvis: every row equal to
    calls of fewer rows, the boundary rows bit-identical to the oracle."""
    from oracle import indexer as oidx
    from smla import indexer as sidx
    from smla import workloads as wl
    S, Hi, Di, N = 66000, 64, 64, 300
    announce(f"long indexer S={S} Hi={Hi} Di={Di} N={N} fp8 keys")
    gc = torch.Generator().manual_seed(6)
    codes, ks = wl.quant_e4m3_pow2(torch.randn(1, N, Di, generator=gc), block=Di)
    ks = ks.reshape(1, N)
    g = torch.Generator(device=dev).manual_seed(6)
    q = torch.randn(1, S, Hi, Di, generator=g, device=dev).to(torch.bfloat16)
    w = torch.randn(1, S, Hi, generator=g, device=dev)
    nvis = torch.randint(0, N + 1, (1, S), generator=g, device=dev, dtype=torch.int32)
    cd, ksd = codes.to(dev), ks.to(dev)
    out = sidx.indexer_score(q, cd, ksd, w, nvis)
    for lo, hi in ((0, 40000), (40000, S)):
        part = sidx.indexer_score(q[:, lo:hi].contiguous(), cd, ksd, w[:, lo:hi].contiguous(),
                                  nvis[:, lo:hi].contiguous())
        torch.cuda.synchronize()
        assert torch.equal(_f32_bits(out[:, lo:hi]), _f32_bits(part)), f"rows {lo}..{hi}"
    rows = _rows_near(S, [CHUNK])
    ref = oidx.indexer_score(q[0, rows].float().cpu().numpy(), codes[0].view(torch.float8_e4m3fn).float().numpy(),
                             ks[0].numpy(), w[0, rows].cpu().numpy(), nvis[0, rows].cpu().numpy())
    assert torch.equal(_f32_bits(out[0, rows].cpu()), _f32_bits(torch.from_numpy(ref)))


def test_indexer_whole_sequences_fp4(dev):
    """Indexer scores for three sequences of 30000 query rows (launches of two sequences, then
    one: keys, block scales and key scales offset per chunk), 16 heads (the vector-ALU kernel),
    fp32 q, keys in the stored fp4 form."""
    from oracle import indexer as oidx
    from oracle import qat
    from smla import indexer as sidx
    B, S, Hi, Di, N = 3, 30000, 16, 64, 200
    announce(f"long indexer B={B} S={S} Hi={Hi} N={N} fp4 keys")
    gc = torch.Generator().manual_seed(7)
    codes, scales = qat.fp4_quantize(qat.hadamard_rotate(torch.randn(B, N, Di, generator=gc).numpy()))
    kvals = qat.fp4_dequantize(codes, scales)
    ks = torch.rand(B, N, generator=gc) + 0.5
    g = torch.Generator(device=dev).manual_seed(7)
    q = torch.randn(B, S, Hi, Di, generator=g, device=dev)
    w = torch.randn(B, S, Hi, generator=g, device=dev)
    nvis = torch.randint(0, N + 1, (B, S), generator=g, device=dev, dtype=torch.int32)
    cd, sd, ksd = torch.from_numpy(codes).to(dev), torch.from_numpy(scales).to(dev), ks.to(dev)
    out = sidx.indexer_score_fp4(q, cd, sd, ksd, w, nvis)
    for b in range(B):
        part = sidx.indexer_score_fp4(q[b:b + 1].contiguous(), cd[b:b + 1].contiguous(), sd[b:b + 1].contiguous(),
                                      ksd[b:b + 1].contiguous(), w[b:b + 1].contiguous(), nvis[b:b + 1].contiguous())
        torch.cuda.synchronize()
        assert torch.equal(_f32_bits(out[b:b + 1]), _f32_bits(part)), f"sequence {b}"
    rows = _rows_near(S, [])
    for b in (1, 2):
        ref = oidx.indexer_score(q[b, rows].cpu().numpy(), kvals[b], ks[b].numpy(), w[b, rows].cpu().numpy(),
                                 nvis[b, rows].cpu().numpy())
        assert torch.equal(_f32_bits(out[b, rows].cpu()), _f32_bits(torch.from_numpy(ref))), f"sequence {b}"


def test_index_decode_pieces_of_one_sequence(dev):
    """Indexer scores and the decode index build in one call over 66000 query rows of one
    sequence: equal to the scores followed by the selection."""
    from smla import indexer as sidx
    from smla import workloads as wl
    S, Hi, Di, N, k, window, n_raw = 66000, 64, 64, 512, 64, 16, 4096
    announce(f"long index_decode S={S} N={N} k={k}")
    gc = torch.Generator().manual_seed(8)
    codes, ks = wl.quant_e4m3_pow2(torch.randn(1, N, Di, generator=gc), block=Di)
    cd, ksd = codes.to(dev), ks.reshape(1, N).to(dev)
    g = torch.Generator(device=dev).manual_seed(8)
    q = torch.randn(1, S, Hi, Di, generator=g, device=dev).to(torch.bfloat16)
    w = torch.randn(1, S, Hi, generator=g, device=dev)
    nvis = torch.randint(1, N + 1, (1, S), generator=g, device=dev, dtype=torch.int32)
    pos = torch.randint(0, n_raw, (S,), generator=g, device=dev, dtype=torch.int32)
    fused = sidx.index_decode(q, cd, ksd, w, nvis, k, pos, window, n_raw)
    sc = sidx.indexer_score(q, cd, ksd, w, nvis)
    two = sidx.select_decode_indices(sc[0], k, pos, window, n_raw, nvis=nvis[0])
    torch.cuda.synchronize()
    assert torch.equal(fused, two)
