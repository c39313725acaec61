"""Pins oracle.compressor against the reference's goldens, brute force and special cases."""
import os

import numpy as np
import torch

from conftest import GOLDEN
from oracle import compressor as oc
from oracle import norm_rope as nr


def test_overlap_transform_golden():
    g = np.load(os.path.join(GOLDEN, "overlap.npz"))
    t = torch.from_numpy(g["t"])
    np.testing.assert_array_equal(oc.overlap_transform(t, 4, 8, 0).numpy(), g["zero"])
    np.testing.assert_array_equal(oc.overlap_transform(t, 4, 8, float("-inf")).numpy(), g["ninf"])


def _case(g, name):
    keys = [k.split("__", 1)[1] for k in g.files if k.startswith(name + "__")]
    return {k: torch.from_numpy(g[f"{name}__{k}"]) for k in keys}


def test_compressor_prefill_golden_outputs_and_state():
    g = np.load(os.path.join(GOLDEN, "compressor.npz"))
    for name in ("small_rem", "small_even", "wide_rem"):
        c = _case(g, name)
        b, s, dim, d, rd = [int(v) for v in c["dims"]]
        kv, state = oc.compressor_prefill(c["x"], c["wkv"], c["wgate"], c["ape"], c["norm_w"], head_dim=d,
                                          ratio=4, rope_head_dim=rd)
        np.testing.assert_allclose(kv.numpy(), c["kv"].numpy(), rtol=1e-5, atol=1e-5)
        ref_state = {k[6:] for k in c if k.startswith("state_")}
        assert set(state) == ref_state, name
        for k in state:
            np.testing.assert_allclose(state[k].numpy(), c["state_" + k].numpy(), rtol=1e-6, atol=1e-6)


def _bruteforce_pool(kv, score, ape, ratio, d):
    """Per (group, channel) loop in float64."""
    b, n, _ = kv.shape
    G = n // ratio
    out = np.zeros((b, G, d))
    kv, score, ape = kv.double().numpy(), score.double().numpy(), ape.double().numpy()
    for bb in range(b):
        for gi in range(G):
            for c in range(d):
                vs, ss = [], []
                if gi > 0:
                    for j in range(ratio):
                        vs.append(kv[bb, (gi - 1) * ratio + j, c])
                        ss.append(score[bb, (gi - 1) * ratio + j, c] + ape[j, c])
                for j in range(ratio):
                    vs.append(kv[bb, gi * ratio + j, d + c])
                    ss.append(score[bb, gi * ratio + j, d + c] + ape[j, d + c])
                ss = np.array(ss)
                w = np.exp(ss - ss.max())
                out[bb, gi, c] = (w * np.array(vs)).sum() / w.sum()
    return out


def test_pool_bruteforce_and_special_cases():
    torch.manual_seed(3)
    b, n, d, r = 2, 12, 6, 4
    kv = torch.randn(b, n, 2 * d)
    sc = torch.randn(b, n, 2 * d)
    ape = torch.randn(r, 2 * d)
    pooled = oc._pool(kv, (sc.reshape(b, n // r, r, 2 * d) + ape).reshape(b, n, 2 * d), r, d)
    np.testing.assert_allclose(pooled.double().numpy(), _bruteforce_pool(kv, sc, ape, r, d), rtol=1e-5, atol=1e-6)
    # uniform scores: mean over the valid slots (4 for group 0, 8 otherwise)
    zero = torch.zeros(b, n, 2 * d)
    pooled = oc._pool(kv, zero, r, d)
    g0 = kv[:, :r, d:].mean(1)
    np.testing.assert_allclose(pooled[:, 0].numpy(), g0.numpy(), rtol=1e-6, atol=1e-6)
    g1 = torch.cat([kv[:, 0:r, :d], kv[:, r:2 * r, d:]], 1).mean(1)
    np.testing.assert_allclose(pooled[:, 1].numpy(), g1.numpy(), rtol=1e-6, atol=1e-6)


def test_ring_reproduces_prefill_rows():
    torch.manual_seed(4)
    d, rd, r, n = 16, 4, 4, 24
    kvp = torch.randn(n, 2 * d)
    scp = torch.randn(n, 2 * d)
    ape = torch.randn(r, 2 * d)
    norm_w = 1 + 0.1 * torch.randn(d)
    freqs = nr.precompute_freqs(rd, n, 65536, 160000.0, 16, 32, 1)
    cis = nr.precompute_freqs_cis(rd, n, 65536, 160000.0, 16, 32, 1)
    pre = oc.gated_pool(kvp[None], scp[None], ape, norm_w, cis, r, rd)[0]
    # prefill the first 8 tokens, then run the ring over the rest
    kvs, scs = oc.ring_init(kvp[:8], scp[:8], ape, r)
    rows = []
    for p in range(8, n):
        row = oc.ring_step(kvs, scs, kvp[p], scp[p], p, ape, norm_w, freqs, r, rd, fp8_sim=False)
        if row is not None:
            rows.append(row)
    np.testing.assert_allclose(torch.stack(rows).numpy(), pre[2:].numpy(), rtol=1e-5, atol=1e-5)


def test_mean_pool_closed_form():
    x = torch.arange(2 * 8 * 3, dtype=torch.float32).reshape(2, 8, 3)
    m = oc.mean_pool(x, 4)
    np.testing.assert_array_equal(m.numpy(), x.reshape(2, 2, 4, 3).mean(2).numpy())
