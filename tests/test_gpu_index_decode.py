"""GPU parity of smla_index_decode (indexer scores + decode index build in one call).

The output must equal, bit for bit, the oracle's fixed-order indexer scores followed by its exact
top-k (window ids first, compressed ids offset by n_raw), with either flag value, over rows with
equal scores and overflow, and for shapes without the 64 x 64 matrix-core form.  Near-ties are
built on purpose: duplicated keys (exact ties broken by index) and key pairs one e4m3 code apart."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import indexer as oidx

pytestmark = pytest.mark.gpu


def _oracle_ids(q, kvals, ks, w, nvis, k, pos, window, n_raw):
    B, S = q.shape[:2]
    rows = []
    for b in range(B):
        sc = oidx.indexer_score(q[b].float().numpy(), kvals[b].numpy(), None if ks is None else ks[b].numpy(),
                                w[b].numpy(), nvis[b].numpy())
        sel = oidx.topk(sc, k, nvis[b].numpy())
        for s in range(S):
            ids = np.where(sel[s] >= 0, sel[s] + n_raw, -1)
            if window:
                win = int(pos[b * S + s]) - window + 1 + np.arange(window)
                win[win < 0] = -1
                ids = np.concatenate([win, ids])
            rows.append(ids)
    return np.stack(rows).astype(np.int32)


def _keys(kind, B, N, Di, g):
    from smla import workloads as wl
    kf = torch.randn(B, N, Di, generator=g)
    if kind == "dup":        # groups of 8 identical keys: exact ties at the boundary
        kf = kf[:, torch.arange(N) // 8 * 8]
    elif kind == "equal":    # every key the same: one score for the whole row
        kf = kf[:, :1].expand(B, N, Di).contiguous()
    codes, scales = wl.quant_e4m3_pow2(kf, block=Di)
    codes = codes.clone()
    scales = scales.reshape(B, N).clone()
    if kind == "near":       # key 2m+1 = key 2m with dim 0 one code apart
        c0 = codes[:, 0::2, 0].clone()
        flip = (c0 & 0x7f) < 0x7e
        codes[:, 1::2] = codes[:, 0::2]
        codes[:, 1::2, 0] = torch.where(flip, c0 ^ 1, c0)
        scales[:, 1::2] = scales[:, 0::2]
    kvals = codes.view(torch.float8_e4m3fn).float()
    return codes, scales, kvals


@pytest.mark.parametrize("B,S,N,k,window,kind,use_scale", [
    (8, 1, 8192, 2048, 128, "random", True),     # the decode_32k index build
    (2, 3, 1000, 300, 0, "random", False),       # several query rows per sequence, ragged N
    (1, 1, 16384, 2048, 128, "random", True),    # 16 scores per thread
    (4, 1, 8192, 2048, 128, "dup", True),
    (4, 1, 8192, 2048, 128, "near", True),
    (2, 1, 4096, 1000, 16, "equal", True),       # spread 0: rescored in full
    (2, 1, 4096, 1000, 16, "overflow", True),    # +-inf scores: rescored in full
])
def test_index_decode_vs_oracle(dev, B, S, N, k, window, kind, use_scale):
    from smla import indexer as sidx
    announce(f"index_decode B={B} S={S} N={N} k={k} window={window} kind={kind}")
    g = torch.Generator().manual_seed(N + B + k)
    Hi = Di = 64
    q = torch.randn(B, S, Hi, Di, generator=g).to(torch.bfloat16)
    w = torch.randn(B, S, Hi, generator=g)
    codes, ks, kvals = _keys(kind, B, N, Di, g)
    if kind == "overflow":
        ks[:, 5] = 3e38
        ks[:, 77] = 3e38
    if not use_scale:
        ks = None
    nvis = torch.full((B, S), N, dtype=torch.int32)
    if B * S > 1:
        nvis.view(-1)[1] = int(N * 0.6)
    if B * S > 3:
        nvis.view(-1)[2] = k // 2      # fewer visible than k: take all
        nvis.view(-1)[3] = 0
    n_raw = 4 * N
    pos = torch.randint(0, n_raw, (B * S,), generator=g, dtype=torch.int32)
    pos[0] = 5                         # window partly before the sequence start
    out = sidx.index_decode(q.to(dev), codes.to(dev), None if ks is None else ks.to(dev), w.to(dev), nvis.to(dev),
                            k, pos.to(dev), window, n_raw)
    ref = _oracle_ids(q, kvals, ks, w, nvis, k, pos.numpy(), window, n_raw)
    np.testing.assert_array_equal(out.cpu().numpy(), ref)


@pytest.mark.parametrize("kind", ["random", "near"])
def test_index_decode_exact_flag(dev, kind):
    """SMLA_INDEX_EXACT gives the same list (the scores are always the fixed-order ones)."""
    from smla import _lib
    from smla import indexer as sidx
    announce(f"index_decode exact flag kind={kind}")
    g = torch.Generator().manual_seed(3)
    B, N, k, window = 2, 4096, 1024, 64
    q = torch.randn(B, 1, 64, 64, generator=g).to(torch.bfloat16)
    w = torch.randn(B, 1, 64, generator=g)
    codes, ks, kvals = _keys(kind, B, N, 64, g)
    nvis = torch.tensor([[N], [N - 100]], dtype=torch.int32)
    pos = torch.tensor([9000, 70], dtype=torch.int32)
    out = sidx.index_decode(q.to(dev), codes.to(dev), ks.to(dev), w.to(dev), nvis.to(dev), k, pos.to(dev),
                            window, 4 * N, flags=_lib.INDEX_EXACT)
    torch.cuda.synchronize()
    ref = _oracle_ids(q, kvals, ks, w, nvis, k, pos.numpy(), window, 4 * N)
    np.testing.assert_array_equal(out.cpu().numpy(), ref)


def test_index_decode_matches_two_step(dev):
    """The one-call form and indexer_score + select_decode_indices agree on the decode_32k step,
    and on a shape outside the 64 x 64 matrix-core form (32 heads, fp32 q)."""
    from smla import indexer as sidx
    from smla import workloads as wl
    announce("index_decode vs two-step")
    w32 = wl.decode_32k()
    B, N = w32["k_codes"].shape[:2]
    nvis = torch.full((B, 1), N, dtype=torch.int32, device=dev)
    pos = torch.full((B,), w32["pos"], dtype=torch.int32, device=dev)
    q, codes, ks, w = (w32[x].to(dev) for x in ("q_idx", "k_codes", "kscale", "w"))
    fused = sidx.index_decode(q, codes, ks, w, nvis, w32["k"], pos, w32["window"], 32768)
    sc = sidx.indexer_score(q, codes, ks, w, nvis)
    two = sidx.select_decode_indices(sc[:, 0], w32["k"], pos, w32["window"], 32768)
    assert torch.equal(fused, two)
    # 32 heads, fp32 q
    g = torch.Generator().manual_seed(4)
    q2 = torch.randn(2, 1, 32, 64, generator=g)
    w2 = torch.randn(2, 1, 32, generator=g)
    codes2, ks2, kv2 = _keys("random", 2, 3000, 64, g)
    nv2 = torch.tensor([[3000], [2500]], dtype=torch.int32)
    pos2 = torch.tensor([100, 5000], dtype=torch.int32)
    out2 = sidx.index_decode(q2.to(dev), codes2.to(dev), ks2.to(dev), w2.to(dev), nv2.to(dev), 700, pos2.to(dev),
                             32, 12000)
    ref2 = _oracle_ids(q2, kv2, ks2, w2, nv2, 700, pos2.numpy(), 32, 12000)
    np.testing.assert_array_equal(out2.cpu().numpy(), ref2)
