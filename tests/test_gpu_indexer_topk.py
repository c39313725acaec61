"""GPU parity of the indexer score (bit-exact to the canonical chain), top-k (exact sets) and the
window index builders."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import indexer as oidx
from oracle import sparse_attn as osa

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("qdt,kdt,use_scale,Hi,Di,N", [
    ("f32", "f32", False, 16, 64, 4096),
    ("bf16", "fp8", True, 64, 64, 8192),
    ("bf16", "bf16", False, 8, 128, 1000),
    ("f32", "fp8", True, 3, 32, 333),
    ("bf16", "f32", True, 64, 64, 257),
    ("f32", "bf16", False, 64, 64, 1000),
    ("f32", "fp8", True, 64, 64, 130),
])
def test_indexer_bit_exact(dev, qdt, kdt, use_scale, Hi, Di, N):
    from smla import indexer as sidx
    from smla import workloads as wl
    announce(f"indexer q={qdt} k={kdt} scale={use_scale} Hi={Hi} Di={Di} N={N}")
    g = torch.Generator().manual_seed(N + Hi)
    B, S = 2, 2
    q = torch.randn(B, S, Hi, Di, generator=g)
    if qdt == "bf16":
        q = q.to(torch.bfloat16)
    kf = torch.randn(B, N, Di, generator=g)
    if kdt == "fp8":
        keys, _ = wl.quant_e4m3_pow2(kf, block=Di)
        kvals = keys.view(torch.float8_e4m3fn).float()
    elif kdt == "bf16":
        keys = kf.to(torch.bfloat16)
        kvals = keys.float()
    else:
        keys = kf
        kvals = kf
    ks = (torch.rand(B, N, generator=g) + 0.5) if use_scale else None
    w = torch.randn(B, S, Hi, generator=g)
    nvis = torch.randint(0, N + 1, (B, S), generator=g, dtype=torch.int32)
    nvis[0, 0] = N
    out = sidx.indexer_score(q.to(dev), keys.to(dev), None if ks is None else ks.to(dev), w.to(dev), nvis.to(dev))
    out = out.cpu().numpy()
    for b in range(B):
        ref = oidx.indexer_score(q[b].float().numpy(), kvals[b].numpy(), None if ks is None else ks[b].numpy(),
                                 w[b].numpy(), nvis[b].numpy())
        np.testing.assert_array_equal(_bits(out[b]), _bits(ref))


def _same(a, b):
    """Bit-identical, except that any NaN matches any NaN (the payload of a NaN made by inf - inf
    differs between the GPU and the host)."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a)
    np.testing.assert_array_equal(nan, np.isnan(b))
    np.testing.assert_array_equal(_bits(a)[~nan], _bits(b)[~nan])


@pytest.mark.parametrize("qdt,use_scale,Hi,Di,N,edges", [
    ("bf16", True, 64, 64, 8192, False),   # two keys per lane, 16 heads per wave
    ("bf16", False, 64, 64, 100, True),    # one key per lane, 8 heads per wave
    ("f32", True, 64, 64, 1000, True),
    ("f32", False, 16, 64, 700, True),     # generic kernel
    ("bf16", True, 8, 128, 1000, False),
    ("f32", True, 3, 32, 333, True),
    ("bf16", True, 100, 64, 300, True),    # more than 64 heads: one thread per key
])
def test_indexer_fp4_bit_exact(dev, qdt, use_scale, Hi, Di, N, edges):
    """Keys in the stored fp4 form (packed e2m1 codes + ue8m0 per 32), the rotation + fp4 of the
    indexer compressor, scored bit-identically to the oracle chain over the decoded keys.  With
    ``edges``, some key blocks carry every code under the extreme scale bytes (0, 1: subnormal
    products; 2 and 252: the ends of the converter's range; 253, 254: overflow; 255: NaN)."""
    from oracle import qat
    from smla import indexer as sidx
    announce(f"indexer fp4 q={qdt} scale={use_scale} Hi={Hi} Di={Di} N={N} edges={edges}")
    g = torch.Generator().manual_seed(3 * N + Hi)
    B, S = 2, 2
    q = torch.randn(B, S, Hi, Di, generator=g)
    if qdt == "bf16":
        q = q.to(torch.bfloat16)
    kf = torch.randn(B, N, Di, generator=g).numpy() * np.exp2(
        torch.randint(-20, 20, (B, N, 1), generator=g).numpy()).astype(np.float32)
    codes, scales = qat.fp4_quantize(qat.hadamard_rotate(kf))
    if edges:
        rng = np.random.default_rng(N)
        rows = rng.choice(N, size=min(N, 40), replace=False)
        for i, r in enumerate(rows):
            codes[i % B, r] = rng.integers(0, 256, Di // 2, dtype=np.uint8)
            codes[i % B, r, :16] = np.arange(0, 256, 17, dtype=np.uint8)  # every code in both nibbles
            scales[i % B, r] = [0, 1, 2, 252, 253, 254, 255, 127][i % 8]
    kvals = qat.fp4_dequantize(codes, scales)
    ks = (torch.rand(B, N, generator=g) + 0.5) if use_scale else None
    w = torch.randn(B, S, Hi, generator=g)
    nvis = torch.randint(0, N + 1, (B, S), generator=g, dtype=torch.int32)
    nvis[0, 0] = N
    out = sidx.indexer_score_fp4(q.to(dev), torch.from_numpy(codes).to(dev), torch.from_numpy(scales).to(dev),
                                 None if ks is None else ks.to(dev), w.to(dev), nvis.to(dev)).cpu().numpy()
    for b in range(B):
        ref = oidx.indexer_score(q[b].float().numpy(), kvals[b], None if ks is None else ks[b].numpy(),
                                 w[b].numpy(), nvis[b].numpy())
        _same(out[b], ref)


def test_indexer_key_path_end_to_end(dev):
    """fp32 compressed keys -> Hadamard + fp4 on the GPU (smla_rotate_fp4, stored form) -> fp4
    scores -> top-2048, against the oracle's rotate_fp4 -> score -> top-k on the same keys; the
    fp4 scores also equal the fp32-key scorer's on the GPU's own round trip."""
    from oracle import qat
    from smla import indexer as sidx
    from smla import qat as sqat
    announce("indexer key path: rotate_fp4 -> indexer_score_fp4 -> topk, B=2 N=8192")
    g = torch.Generator().manual_seed(11)
    B, N, Hi, Di, k = 2, 8192, 64, 64, 2048
    kf = torch.randn(B, N, Di, generator=g)
    q = torch.randn(B, 1, Hi, Di, generator=g).to(torch.bfloat16)
    w = torch.randn(B, 1, Hi, generator=g)
    ks = torch.rand(B, N, generator=g) + 0.5
    nvis = torch.tensor([[N], [5000]], dtype=torch.int32)
    codes, scales = sqat.fp4_pack(kf.to(dev), rotate=True)
    sc = sidx.indexer_score_fp4(q.to(dev), codes, scales, ks.to(dev), w.to(dev), nvis.to(dev))
    ids = sidx.topk(sc[:, 0], k, nvis[:, 0].to(dev)).cpu().numpy()
    sc_rt = sidx.indexer_score(q.to(dev), sqat.rotate_fp4(kf.to(dev)), ks.to(dev), w.to(dev), nvis.to(dev))
    _same(sc.cpu().numpy(), sc_rt.cpu().numpy())
    for b in range(B):
        ref = oidx.indexer_score(q[b].float().numpy(), qat.rotate_fp4(kf[b].numpy()), ks[b].numpy(), w[b].numpy(),
                                 nvis[b].numpy())
        _same(sc[b].cpu().numpy(), ref)
        np.testing.assert_array_equal(ids[b], oidx.topk(ref, k, nvis[b].numpy())[0])


@pytest.mark.parametrize("R,N,k,ties", [
    (1, 100, 10, False), (3, 1024, 512, True), (2, 1025, 1000, True), (8, 8192, 2048, False),
    (8, 8192, 2048, True), (1, 16384, 2048, True), (2, 65536, 2048, False), (4, 3000, 1, True),
    (2, 50000, 7000, True)])
def test_topk_exact(dev, R, N, k, ties):
    from smla import indexer as sidx
    announce(f"topk R={R} N={N} k={k} ties={ties}")
    rng = np.random.default_rng(N + k)
    if ties:
        s = (rng.integers(-40, 41, (R, N)) * 0.25).astype(np.float32)
        s[s == 0] = np.where(rng.random((s == 0).sum()) < 0.5, -0.0, 0.0).astype(np.float32)
    else:
        s = rng.standard_normal((R, N)).astype(np.float32)
    nvis = rng.integers(0, N + 1, R).astype(np.int32)
    nvis[0] = N
    if R > 1:
        nvis[1] = min(k, N)           # exactly k visible
    got = sidx.topk(torch.from_numpy(s).to(dev), k, torch.from_numpy(nvis).to(dev)).cpu().numpy()
    np.testing.assert_array_equal(got, oidx.topk(s, k, nvis))
    got0 = sidx.topk(torch.from_numpy(s).to(dev), k, id_offset=5).cpu().numpy()
    ref0 = oidx.topk(s, k)
    np.testing.assert_array_equal(got0, np.where(ref0 >= 0, ref0 + 5, -1))


def test_topk_into_strided_view(dev):
    """ops.topk_into writes the same selection into a column slice of a wider int32 buffer (its
    row stride), leaving the other columns alone."""
    from smla import indexer as sidx
    from smla import ops
    announce("topk_into strided view R=4 N=3000 k=700")
    g = torch.Generator().manual_seed(21)
    sc = torch.randn(4, 3000, generator=g).to(dev)
    nvis = torch.tensor([3000, 10, 700, 2500], dtype=torch.int32, device=dev)
    buf = torch.full((4, 900), -7, dtype=torch.int32, device=dev)
    ops.topk_into(sc, 700, buf[:, 100:800], id_offset=5, nvis=nvis)
    ref = sidx.topk(sc, 700, nvis, id_offset=5)
    torch.testing.assert_close(buf[:, 100:800], ref, rtol=0, atol=0)
    assert (buf[:, :100] == -7).all() and (buf[:, 800:] == -7).all()


def test_topk_all_equal_and_ragged(dev):
    from smla import indexer as sidx
    announce("topk all equal")
    s = np.zeros((2, 5000), np.float32)
    s[1, ::2] = -0.0
    got = sidx.topk(torch.from_numpy(s).to(dev), 300).cpu().numpy()
    np.testing.assert_array_equal(got, np.tile(np.arange(300, dtype=np.int32), (2, 1)))


@pytest.mark.parametrize("w,bsz,seqlen,start_pos", [
    (128, 2, 1, 32767), (8, 1, 1, 9), (8, 3, 1, 3), (128, 1, 1, 1), (8, 2, 5, 0), (128, 1, 300, 0)])
def test_window_idxs(dev, w, bsz, seqlen, start_pos):
    from smla import sparse_attn as ssa
    announce(f"window idx w={w} start={start_pos}")
    got = ssa.get_window_topk_idxs(w, bsz, seqlen, start_pos, device=dev).cpu()
    ref = osa.get_window_topk_idxs(w, bsz, seqlen, start_pos)
    assert got.shape == ref.shape
    np.testing.assert_array_equal(got.numpy(), ref.numpy())


def test_decode_window_idxs(dev):
    from smla import ops
    announce("decode window idx")
    pos = torch.tensor([0, 5, 127, 128, 32767], dtype=torch.int32, device=dev)
    got = ops.decode_window_idxs(pos, 128).cpu().numpy()
    for r, p in enumerate([0, 5, 127, 128, 32767]):
        ref = np.arange(p - 127, p + 1)
        ref[ref < 0] = -1
        np.testing.assert_array_equal(got[r], ref)


@pytest.mark.parametrize("case", ["outlier", "inf", "nan", "crowded"])
def test_topk_fallback_spreads(dev, case):
    """Rows whose value spread defeats the bucket pass (one huge outlier, infinities, NaN, more
    than 256 entries sharing the boundary bucket) take the radix path; sets stay exact."""
    from smla import indexer as sidx
    announce(f"topk fallback {case}")
    rng = np.random.default_rng(7)
    R, N, k = 3, 8192, 2048
    s = rng.standard_normal((R, N)).astype(np.float32)
    if case == "outlier":
        s[:, 17] = 3.0e38
    elif case == "inf":
        s[:, ::97] = np.inf
        s[:, 5::89] = -np.inf
    elif case == "nan":
        s[:, ::101] = np.nan
        s[1, 3::53] = -np.nan
    else:
        s = (rng.integers(0, 4, (R, N)) * 1e-3).astype(np.float32)
        s[:, 0] = 1.0e6
    nvis = np.array([N, N - 100, 3000], np.int32)
    got = sidx.topk(torch.from_numpy(s).to(dev), k, torch.from_numpy(nvis).to(dev)).cpu().numpy()
    np.testing.assert_array_equal(got, oidx.topk(s, k, nvis))


@pytest.mark.parametrize("case", ["tail", "scattered", "few_finite", "all_neg_inf"])
def test_topk_negative_infinity_scores(dev, case):
    """-inf is the indexer's mark of masked keys: rows that hold -inf scores as visible entries keep
    the bucket pass when k finite scores remain (the -inf entries are never selected), and take the
    exact fallback when fewer remain (the -inf entries are then taken lowest index first)."""
    from smla import indexer as sidx
    announce(f"topk -inf {case}")
    rng = np.random.default_rng(11)
    R, N, k = 3, 16384, 2048
    s = (rng.standard_normal((R, N)) * 40).astype(np.float32)
    if case == "tail":
        s[:, N - 5:] = -np.inf
    elif case == "scattered":
        s[:, ::7] = -np.inf
    elif case == "few_finite":
        s[:, 1500:] = -np.inf              # 1500 finite scores: every one selected, then -inf by index
    else:
        s[:] = -np.inf
    got = sidx.topk(torch.from_numpy(s).to(dev), k).cpu().numpy()
    np.testing.assert_array_equal(got, oidx.topk(s, k))
    nvis = np.array([N, N - 3, 9000], np.int32)
    got = sidx.topk(torch.from_numpy(s).to(dev), k, torch.from_numpy(nvis).to(dev)).cpu().numpy()
    np.testing.assert_array_equal(got, oidx.topk(s, k, nvis))


@pytest.mark.parametrize("R,N,k,window", [(8, 8192, 2048, 128), (3, 100, 512, 128), (2, 4096, 64, 7)])
def test_select_decode_fused(dev, R, N, k, window):
    """One launch writes the decode window ids then the top-k ids (offset into the raw cache)."""
    from smla import indexer as sidx
    announce(f"select_decode R={R} N={N} k={k} window={window}")
    rng = np.random.default_rng(R * N + k)
    s = rng.standard_normal((R, N)).astype(np.float32)
    pos = rng.integers(0, 4 * N, R).astype(np.int32)
    pos[0] = 3
    n_raw = 4 * N + 1
    got = sidx.select_decode_indices(torch.from_numpy(s).to(dev), k, torch.from_numpy(pos).to(dev), window,
                                     n_raw).cpu().numpy()
    assert got.shape == (R, window + k)
    sel = oidx.topk(s, k)
    for r in range(R):
        win = np.arange(pos[r] - window + 1, pos[r] + 1)
        win[win < 0] = -1
        np.testing.assert_array_equal(got[r, :window], win)
        np.testing.assert_array_equal(got[r, window:], np.where(sel[r] >= 0, sel[r] + n_raw, -1))
