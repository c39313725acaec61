"""GPU parity of smla_decode_attn: the decode index build over indexer scores (window ids of pos,
then the top-k of the first nvis scores, ascending, offset by n_raw) and the attention over it in
one call.  Its output must equal, bit for bit, smla_select_decode followed by the two-source
attention with the default split plan -- with the selection run inside the attention workgroups
(bf16 rows, short splits, N <= 18432) and on the list path (other shapes) -- and the oracle within
the bf16 tolerance.  Cases: the decode_32k step, take-all rows (nvis <= k), -inf scores, equal
scores, early positions (negative window ids), N not a multiple of 4, 16384 scores, two head
groups, several query rows per sequence."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import sparse_attn as osa

pytestmark = pytest.mark.gpu


def _two_step(q, raw, comp, sink, sc, pos, window, k, scale, nvis):
    from smla import indexer as sidx
    from smla import sparse_attn as ssa
    B, S = q.shape[:2]
    idx = sidx.select_decode_indices(sc, k, pos, window, raw.shape[1], nvis=nvis)   # [B*S, window + k]
    return ssa.sparse_attn_two_source(q, raw, comp, sink, idx.view(B, S, -1), scale, dv=512), idx


def _case(dev, B, S, H, n_raw, n_comp, N, k, window, pos_list, seed, nvis_list=None, kind="random",
          kv_dtype=torch.bfloat16):
    from smla import sparse_attn as ssa
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, S, H, 576, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    raw = (torch.randn(B, n_raw, 576, generator=g) * 0.5).to(kv_dtype).to(dev)
    comp = (torch.randn(B, n_comp, 576, generator=g) * 0.5).to(kv_dtype).to(dev)
    sc = torch.randn(B * S, N, generator=g)
    if kind == "inf":
        sc[:, ::3] = float("-inf")
    elif kind == "equal":
        sc = torch.full((B * S, N), 0.25)
    elif kind == "ties":
        sc = torch.round(sc * 4) / 4        # many exact ties at the boundary
    sc = sc.to(dev)
    sink = torch.randn(H, generator=g).to(dev)
    pos = torch.tensor(pos_list, dtype=torch.int32, device=dev)
    nvis = None if nvis_list is None else torch.tensor(nvis_list, dtype=torch.int32, device=dev)
    scale = 576 ** -0.5
    out = ssa.decode_attn(q, raw, comp, sink, sc, pos, window, k, scale, dv=512, nvis=nvis)
    ref, idx = _two_step(q, raw, comp, sink, sc, pos, window, k, scale, nvis)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16) if out.dtype == torch.bfloat16 else out,
                       ref.view(torch.int16) if ref.dtype == torch.bfloat16 else ref), "differs from the two-step path"
    return q, raw, comp, sink, idx, out


@pytest.mark.parametrize("B,S,H,n_raw,n_comp,N,k,window,kind,nvis", [
    (8, 1, 64, 2048, 1024, 1024, 256, 128, "random", None),     # in-kernel selection, several splits
    (4, 1, 64, 4096, 2048, 2048, 512, 128, "inf", None),        # -inf scores
    (4, 1, 64, 4096, 2048, 2048, 512, 128, "ties", None),       # exact ties across the boundary
    (2, 1, 64, 4096, 2048, 2048, 512, 128, "equal", None),      # one score for the whole row
    (4, 1, 64, 4096, 2048, 2048, 512, 128, "random", [100, 2048, 511, 513]),  # take-all rows and nvis
    (2, 1, 64, 4096, 1000, 1001, 300, 128, "random", None),     # N % 4 != 0: element loads
    (2, 1, 128, 1024, 512, 512, 128, 64, "random", None),       # two head groups
    (2, 3, 64, 1024, 512, 512, 128, 128, "random", None),       # several query rows per sequence
])
def test_decode_attn_matches_two_step(dev, B, S, H, n_raw, n_comp, N, k, window, kind, nvis):
    announce(f"decode_attn B={B} S={S} H={H} N={N} k={k} window={window} kind={kind} nvis={nvis}")
    R = B * S
    pos = [(n_raw - 1 - 7 * r) for r in range(R)]
    pos[0] = 5  # an early position: most window ids negative
    nv = None if nvis is None else (nvis * S)[:R]
    _case(dev, B, S, H, n_raw, n_comp, N, k, window, pos, seed=N + k + window, nvis_list=nv, kind=kind)


def test_decode_attn_vs_oracle(dev):
    """The one-call result against the fp32 oracle over the list the selection gives."""
    announce("decode_attn vs oracle")
    B, H, n_raw, n_comp, N, k, window = 2, 64, 2048, 1024, 1024, 256, 128
    q, raw, comp, sink, idx, out = _case(dev, B, 1, H, n_raw, n_comp, N, k, window, [2047, 900], seed=1)
    for b in range(B):
        kv = torch.cat([raw[b].float(), comp[b].float()]).cpu()
        ref = osa.sparse_attn(q[b].float().cpu(), kv, sink.cpu(), idx[b:b + 1].cpu(), 576 ** -0.5, dv=512)
        err = (out[b].float().cpu() - ref).abs().max().item()
        assert err <= 1e-2 * max(ref.abs().max().item(), 1e-30) + 2e-3, f"row {b}: max abs {err:.3e}"


def test_decode_attn_decode_32k(dev):
    """The decode_32k step (indexer scores of 8 sequences over 8192 compressed rows, k = 2048,
    window 128) and the 16384-score form of decode_64k."""
    from smla import compressor as scomp
    from smla import indexer as sidx
    from smla import sparse_attn as ssa
    from smla import workloads as wl
    announce("decode_attn decode_32k")
    w = wl.decode_32k()
    raw = w["raw"].to(dev)
    comp = scomp.block_mean_pool(raw, 4)
    q = w["q"].to(dev)
    sc = sidx.indexer_score(w["q_idx"].to(dev), w["k_codes"].to(dev), w["kscale"].to(dev), w["w"].to(dev))[:, 0]
    pos = torch.full((q.shape[0],), w["pos"], dtype=torch.int32, device=dev)
    out = ssa.decode_attn(q, raw, comp, None, sc.contiguous(), pos, w["window"], w["k"], w["scale"], dv=512)
    ref, _ = _two_step(q, raw, comp, None, sc.contiguous(), pos, w["window"], w["k"], w["scale"], None)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    # 16384 scores per row (24 per thread in the workgroup's selection)
    _case(dev, 1, 1, 64, 65536, 16384, 16384, 2048, 128, [65535], seed=9)


def test_decode_attn_list_path(dev):
    """Shapes the in-kernel selection does not take run the list path inside the same entry:
    fp32 rows, and more than 18432 scores."""
    announce("decode_attn list path")
    _case(dev, 2, 1, 64, 1024, 512, 512, 128, 64, [1023, 500], seed=3, kv_dtype=torch.float32)
    _case(dev, 1, 1, 64, 1024, 20000, 20000, 512, 128, [1023], seed=4)


def test_decode_attn_rejects(dev):
    """Argument errors are refused on the host."""
    from smla import _lib
    from smla import sparse_attn as ssa
    q = torch.zeros(1, 1, 64, 576, dtype=torch.bfloat16, device=dev)
    raw = torch.zeros(1, 256, 576, dtype=torch.bfloat16, device=dev)
    comp = torch.zeros(1, 64, 576, dtype=torch.bfloat16, device=dev)
    sc = torch.zeros(1, 64, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        ssa.decode_attn(q, raw, comp, None, torch.zeros(2, 64, device=dev), pos, 128, 32, 0.04)   # rows != B*S
    with pytest.raises(_lib.SmlaError):
        ssa.decode_attn(q, raw, comp, None, sc, pos, 128, 0, 0.04)                             # k = 0
