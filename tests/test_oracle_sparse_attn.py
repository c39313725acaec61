"""Pins oracle.sparse_attn: window-index branches by brute force; attention by a library routine
(scaled_dot_product_attention), closed forms, invariances and a float64 brute-force loop."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import sparse_attn as osa


def _window_bruteforce(w, bsz, seqlen, start_pos):
    if start_pos >= w - 1:
        p = start_pos % w
        row = list(range(p + 1, w)) + list(range(0, p + 1))
        return np.array([[row]] * bsz)
    if start_pos > 0:
        row = list(range(start_pos + 1)) + [-1] * (w - start_pos - 1)
        return np.array([[row]] * bsz)
    cols = min(seqlen, w)
    m = np.full((seqlen, cols), -1)
    for i in range(seqlen):
        lo = max(0, i - w + 1)
        for j in range(cols):
            if lo + j <= i:
                m[i, j] = lo + j
    return np.array([m] * bsz)


@pytest.mark.parametrize("w,bsz,seqlen,start_pos", [
    (8, 2, 1, 7), (8, 1, 1, 9), (8, 3, 1, 100), (128, 1, 1, 32767),   # ring
    (8, 2, 1, 3), (8, 1, 1, 1), (128, 1, 1, 5),                        # partial
    (8, 2, 5, 0), (8, 1, 8, 0), (8, 1, 20, 0), (128, 1, 300, 0)])     # prefill band
def test_window_idxs_all_branches(w, bsz, seqlen, start_pos):
    got = osa.get_window_topk_idxs(w, bsz, seqlen, start_pos).numpy()
    np.testing.assert_array_equal(got, _window_bruteforce(w, bsz, seqlen, start_pos))


def test_engine_decode_idxs():
    ids = osa.engine_decode_idxs(pos=10, n_window_rows=11, n_comp=5, ratio=4).tolist()
    assert ids == list(range(11)) + [11, 12]              # (10+1)//4 = 2 visible compressed rows
    ids = osa.engine_decode_idxs(pos=300, n_window_rows=128, n_comp=75, ratio=4).tolist()
    assert ids == list(range(128)) + [128 + j for j in range(75)]
    assert osa.engine_decode_idxs(pos=300, n_window_rows=128, n_comp=75, ratio=0).tolist() == list(range(128))


def _rand(s=3, h=4, d=12, n=20, T=7, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(s, h, d, generator=g)
    kv = torch.randn(n, d, generator=g)
    idx = torch.randint(0, n, (s, T), generator=g)
    return q, kv, idx


def test_matches_sdpa_without_sink():
    q, kv, idx = _rand(s=5, h=3, d=16, n=40, T=9)
    scale = 0.3
    out = osa.sparse_attn(q, kv, None, idx, scale)
    for i in range(q.shape[0]):
        g = kv[idx[i]]                                           # [T, d]
        ref = F.scaled_dot_product_attention(q[i][:, None, :], g[None].expand(3, -1, -1),
                                             g[None].expand(3, -1, -1), scale=scale)[:, 0]
        np.testing.assert_allclose(out[i].numpy(), ref.numpy(), rtol=1e-5, atol=1e-6)


def test_single_row_closed_form_with_sink():
    q, kv, _ = _rand(s=1, h=4, d=8, n=5)
    sink = torch.tensor([-1.0, 0.0, 2.0, float("-inf")])
    idx = torch.tensor([[3]])
    out = osa.sparse_attn(q, kv, sink, idx, 0.5)
    x = 0.5 * (q[0] @ kv[3])                                      # [h]
    wgt = torch.exp(x) / (torch.exp(x) + torch.exp(sink))
    np.testing.assert_allclose(out[0].numpy(), (wgt[:, None] * kv[3][None]).numpy(), rtol=1e-5, atol=1e-6)


def test_permutation_masking_duplicates():
    q, kv, idx = _rand(s=2, h=2, d=6, n=10, T=6)
    sink = torch.tensor([0.5, -0.3])
    base = osa.sparse_attn(q, kv, sink, idx, 0.7)
    perm = idx[:, torch.randperm(6, generator=torch.Generator().manual_seed(1))]
    np.testing.assert_allclose(osa.sparse_attn(q, kv, sink, perm, 0.7).numpy(), base.numpy(), rtol=1e-6, atol=1e-7)
    # -1 entries behave as if removed
    padded = torch.cat([idx, torch.full((2, 3), -1)], 1)
    np.testing.assert_allclose(osa.sparse_attn(q, kv, sink, padded, 0.7).numpy(), base.numpy(), rtol=1e-6, atol=1e-7)
    # a duplicated id counts twice: equal to a kv with that row copied
    dup = torch.cat([idx, idx[:, :1]], 1)
    kv2 = torch.cat([kv, kv[idx[0, 0]][None]])
    alt = torch.cat([idx, torch.full((2, 1), 10)], 1)
    a = osa.sparse_attn(q[:1], kv, sink, dup[:1], 0.7)
    b = osa.sparse_attn(q[:1], kv2, sink, alt[:1], 0.7)
    np.testing.assert_allclose(a.numpy(), b.numpy(), rtol=1e-6, atol=1e-7)


def test_all_masked_is_nan_and_bruteforce():
    q, kv, idx = _rand(s=3, h=2, d=5, n=9, T=4)
    idx[1] = -1
    sink = torch.tensor([0.2, -1.0])
    out = osa.sparse_attn(q, kv, sink, idx, 0.4)
    assert torch.isnan(out[1]).all() and not torch.isnan(out[0]).any()
    bf = osa.sparse_attn_bruteforce(q, kv, sink, idx, 0.4)
    np.testing.assert_allclose(out[[0, 2]].double().numpy(), bf[[0, 2]].numpy(), rtol=1e-5, atol=1e-7)


def test_value_slice_is_prefix_of_full_output():
    q, kv, idx = _rand(s=2, h=3, d=20, n=15, T=5)
    full = osa.sparse_attn(q, kv, None, idx, 1 / math.sqrt(20))
    part = osa.sparse_attn(q, kv, None, idx, 1 / math.sqrt(20), dv=16)
    np.testing.assert_array_equal(part.numpy(), full[..., :16].numpy())
