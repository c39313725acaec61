"""GPU parity on the long-context decode workload: one sequence, raw latent [65536, 576] and its
block-4 mean pool [16384, 576], fp8 indexer keys [16384, 64], consecutive positions 65516..65535.
Per position p the indexer scores the (p+1)//4 causally visible compressed keys (bit-exact to
the canonical chain), the index list is the window p-127..p followed by the top-2048 (exact
set, ascending), and attention matches the fp32 oracle within the bf16 tolerance."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import indexer as oidx
from oracle import sparse_attn as osa

pytestmark = pytest.mark.gpu

BF16_ABS, BF16_REL = 2e-2, 1e-2


@pytest.fixture(scope="module")
def w64(dev):
    from smla import compressor as scomp
    from smla import workloads as wl
    w = wl.decode_64k()
    raw = w["raw"].to(dev)
    comp = scomp.block_mean_pool(raw, 4)
    kv = torch.cat([raw[0].cpu().float(), comp[0].cpu().float()])   # the oracle's [raw; compressed] rows
    return w, raw, comp, kv


@pytest.mark.parametrize("step", range(20))
def test_decode_64k_step(dev, w64, step):
    from smla import indexer as sidx
    from smla import sparse_attn as ssa
    w, raw, comp, kv = w64
    p = w["pos0"] + step
    nv = (p + 1) // 4
    announce(f"decode_64k step={step} pos={p} visible compressed={nv}")
    n_raw, k, win = raw.shape[1], w["k"], w["window"]
    nvis = torch.tensor([[nv]], dtype=torch.int32, device=dev)
    sc = sidx.indexer_score(w["q_idx"][step][None, None].to(dev), w["k_codes"].to(dev), w["kscale"].to(dev),
                            w["w"][step][None, None].to(dev), nvis)
    idx = sidx.select_decode_indices(sc[:, 0], k, torch.tensor([p], dtype=torch.int32, device=dev), win, n_raw)
    out = ssa.sparse_attn_two_source(w["q"][step][None].to(dev), raw, comp, None, idx[:, None, :], w["scale"], dv=512)
    # indexer: bit-exact over the visible keys, -inf beyond
    sref = oidx.indexer_score(w["q_idx"][step][None].float().numpy(),
                              w["k_codes"][0].view(torch.float8_e4m3fn).float().numpy(),
                              w["kscale"][0].numpy(), w["w"][step][None].numpy(), np.array([nv], np.int32))
    got = sc[0].cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), sref.view(np.uint32))
    # index list: window then the exact top-k of the visible keys
    sel = oidx.topk(sref, k, np.array([nv], np.int32))[0]
    ids_ref = np.concatenate([np.arange(p - win + 1, p + 1), np.where(sel >= 0, sel + n_raw, -1)]).astype(np.int32)
    np.testing.assert_array_equal(idx[0].cpu().numpy(), ids_ref)
    # attention
    ref = osa.sparse_attn(w["q"][step].float(), kv, None, torch.from_numpy(ids_ref)[None], w["scale"], dv=512)
    o = out[0].float().cpu()
    assert not torch.isnan(o).any()
    err = (o - ref).abs().max().item()
    rel = err / max(ref.abs().max().item(), 1e-30)
    assert err <= BF16_ABS and rel <= BF16_REL, f"max abs {err:.3e}, rel {rel:.3e}"
    bad = ((o - ref).abs() > BF16_REL * ref.abs() + 4e-3 * ref.abs().max()).sum().item()
    assert bad == 0, f"{bad} elements outside rel {BF16_REL} + 4e-3 max|ref| (per element)"
