"""GPU parity of the decode-layer wiring (``smla.engine.DecodeLayer``, ``oracle/decode_engine.py:73-119``)
against the oracle's composition (``oracle/engine.py``), at the model's layer shapes (hidden 4096,
q rank 1024, 64 heads x 512, output 8 groups x 1024), for two sequences stepped token by token.

Per step: the layer output (relative L2 error <= 1e-2: every product is a bf16 HIP kernel and the
window and compressed rows are stored in bf16, while the oracle runs float64 products on the same
bf16 weights; measured worst cases are about 5e-3), the window row written at p (rope dims
<= 1e-2) and every emitted compressed row (rope dims <= 2e-2), whose fp8 round-tripped dims are
held to 4e-2.  A wrong position, a missing rotation, a misplaced row or a wrong id list changes
the output by O(1)."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import engine as oe

pytestmark = pytest.mark.gpu


def _make_weights(ratio, seed=7):
    g = torch.Generator().manual_seed(seed)
    bf = lambda *s, sc=0.02: (torch.randn(*s, generator=g) * sc).to(torch.bfloat16)
    f32 = lambda *s, sc=0.1, base=0.0: base + torch.randn(*s, generator=g) * sc
    t = dict(wq_a=bf(1024, 4096), q_a_norm=f32(1024, base=1.0), wq_b=bf(64 * 512, 1024), wkv=bf(512, 4096),
             kv_a_norm=f32(512, base=1.0), wo_a=bf(8 * 1024, 4096), wo_b=bf(4096, 8 * 1024), sinks=f32(64, sc=1.0))
    if ratio == 4:
        t.update(wkv_c=bf(1024, 4096), wgate_c=bf(1024, 4096), ape=f32(4, 1024), norm_c=f32(512, base=1.0))
    return t


def _rel(a, b):
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _check_row(got, ref, tol, what):
    """Rope dims (no fp8) within `tol`; the 448 fp8 round-tripped dims within 4e-2: a bf16-sized
    input difference moves some values across an e4m3 rounding boundary, one step (up to 1/8 of
    the value) each."""
    r = _rel(got[-64:], ref[-64:])
    assert r <= tol, f"{what}: rope dims rel err {r:.3e}"
    n = _rel(got[:-64], ref[:-64])
    assert n <= 4e-2, f"{what}: fp8 dims rel err {n:.3e}"


@pytest.mark.parametrize("ratio,steps", [(4, 136), (0, 24), (128, 24)])
def test_decode_layer_vs_oracle(dev, ratio, steps):
    from smla import engine
    announce(f"decode layer ratio={ratio} steps={steps}")
    t = _make_weights(ratio)
    w = engine.LayerWeights(**{k: v.to(dev) for k, v in t.items()})
    wo = oe.OracleWeights(**{k: (v.double().numpy() if v.dtype == torch.bfloat16 else v.float())
                             for k, v in t.items()})
    B, max_pos = 2, 256
    layer = engine.DecodeLayer(w, B, ratio, max_pos=max_pos, device=dev)
    states = [oe.LayerState(ratio, max_pos=max_pos) for _ in range(B)]
    g = torch.Generator().manual_seed(100 + ratio)
    worst = 0.0
    for p in range(steps):
        xn = torch.randn(B, 4096, generator=g).to(torch.bfloat16)
        pos = torch.full((B,), p, dtype=torch.int32, device=dev)
        y = layer.step(xn.to(dev), pos).float().cpu()
        for b in range(B):
            yr, kv, ids, _ = oe.decode_step(states[b], wo, xn[b].float(), p)
            r = _rel(y[b], yr)
            worst = max(worst, r)
            assert r <= 1e-2, f"step {p} seq {b}: output rel err {r:.3e}"
            _check_row(layer.raw[b, p % 128].float().cpu(), kv, 1e-2, f"step {p} seq {b}: window row")
            if ratio == 4 and (p + 1) % 4 == 0:
                j = (p + 1) // 4 - 1
                assert len(states[b].comp) == j + 1
                _check_row(layer.comp32[b, j].cpu(), states[b].comp[j], 2e-2, f"step {p} seq {b}: compressed row {j}")
    announce(f"worst output rel err {worst:.3e}")


@pytest.mark.parametrize("k,steps", [(8, 72), (40, 200)])
def test_decode_layer_indexer_topk_vs_oracle(dev, k, steps):
    """``step(scores=...)``: the compressed ids are the top-k of the min((p+1)//4, ncap) visible
    slots by (score desc, index asc) instead of all of them.  Positions run from below the point
    where the visible rows exceed k to well above it; scores carry ties, and slots not yet visible
    get the largest scores (a list that ranked them would differ).  Per step the id set equals the
    oracle's exactly and the output is within 1e-2 relative L2."""
    from smla import engine
    announce(f"decode layer indexer top-k k={k} steps={steps}")
    t = _make_weights(4, seed=11)
    w = engine.LayerWeights(**{kk: v.to(dev) for kk, v in t.items()})
    wo = oe.OracleWeights(**{kk: (v.double().numpy() if v.dtype == torch.bfloat16 else v.float())
                             for kk, v in t.items()})
    B, max_pos = 2, 256
    layer = engine.DecodeLayer(w, B, 4, max_pos=max_pos, device=dev)
    states = [oe.LayerState(4, max_pos=max_pos) for _ in range(B)]
    g = torch.Generator().manual_seed(200 + k)
    ncap = max_pos // 4
    for p in range(steps):
        xn = torch.randn(B, 4096, generator=g).to(torch.bfloat16)
        # quantised scores (ties), invisible slots above every visible one
        sc = torch.round(torch.randn(B, ncap, generator=g) * 4) / 4
        nv = min(ncap, (p + 1) // 4)
        sc[:, nv:] = 100.0
        pos = torch.full((B,), p, dtype=torch.int32, device=dev)
        scd = sc.to(dev)
        y = layer.step(xn.to(dev), pos, scores=scd, k=k).float().cpu()
        ids = layer.index_list(pos, scores=scd, k=k).cpu()
        for b in range(B):
            yr, _, ids_ref, _ = oe.decode_step(states[b], wo, xn[b].float(), p, scores=sc[b].numpy(), k=k)
            got = ids[b][ids[b] >= 0].tolist()
            # window ids: ring rows here (position pp at row pp % 128), positions there; compressed
            # ids: 128 + j here, (p + 1) + j there
            got = sorted(p - (p - i) % 128 if i < 128 else (p + 1) + (i - 128) for i in got)
            assert got == sorted(ids_ref.tolist()), f"step {p} seq {b}: id sets differ"
            assert len(ids_ref) == min(p + 1, 128) + min(nv, k)
            r = _rel(y[b], yr)
            assert r <= 1e-2, f"step {p} seq {b}: output rel err {r:.3e}"


@pytest.mark.parametrize("ratio,S,steps", [(4, 37, 6), (4, 140, 5), (0, 30, 3), (128, 133, 3)])
def test_prefill_then_decode_vs_oracle(dev, ratio, S, steps):
    """``DecodeLayer.prefill`` on a prompt of S tokens (a remainder group, a window that wraps past
    128 rows), then ``step`` from position S: every prompt position's output within 1e-2 relative
    L2 of the oracle prefill, the window and compressed rows as in the decode test, and the decode
    steps that follow (which read the ring the prefill set) within 1e-2."""
    from smla import engine
    announce(f"prefill ratio={ratio} S={S} then {steps} steps")
    t = _make_weights(ratio, seed=21)
    w = engine.LayerWeights(**{k: v.to(dev) for k, v in t.items()})
    wo = oe.OracleWeights(**{k: (v.double().numpy() if v.dtype == torch.bfloat16 else v.float())
                             for k, v in t.items()})
    B, max_pos = 2, 256
    layer = engine.DecodeLayer(w, B, ratio, max_pos=max_pos, device=dev)
    states = [oe.LayerState(ratio, max_pos=max_pos) for _ in range(B)]
    g = torch.Generator().manual_seed(300 + S)
    xp = torch.randn(B, S, 4096, generator=g).to(torch.bfloat16)
    y = layer.prefill(xp.to(dev)).float().cpu()
    for b in range(B):
        yr, _, _ = oe.prefill(states[b], wo, xp[b].float())
        for i in range(S):
            r = _rel(y[b, i], yr[i])
            assert r <= 1e-2, f"prefill seq {b} position {i}: output rel err {r:.3e}"
            if i >= S - 128:   # the ring keeps the prompt's last 128 window rows, position i at row i % 128
                _check_row(layer.raw[b, i % 128].float().cpu(), states[b].win[i], 1e-2,
                           f"prefill seq {b}: window row {i}")
        assert len(states[b].comp) == (S // 4 if ratio == 4 else 0)
        for j in range(len(states[b].comp)):
            _check_row(layer.comp32[b, j].cpu(), states[b].comp[j], 2e-2, f"prefill seq {b}: compressed row {j}")
    for p in range(S, S + steps):
        xn = torch.randn(B, 4096, generator=g).to(torch.bfloat16)
        y = layer.step(xn.to(dev), torch.full((B,), p, dtype=torch.int32, device=dev)).float().cpu()
        for b in range(B):
            yr, _, _, _ = oe.decode_step(states[b], wo, xn[b].float(), p)
            r = _rel(y[b], yr)
            assert r <= 1e-2, f"step {p} seq {b}: output rel err {r:.3e}"
            if ratio == 4 and (p + 1) % 4 == 0:
                j = (p + 1) // 4 - 1
                _check_row(layer.comp32[b, j].cpu(), states[b].comp[j], 2e-2, f"step {p} seq {b}: compressed row {j}")


def test_decode_layer_window_ring_wraps(dev):
    """The window ring over 320 decode steps of a ratio-4 layer (the 128-row ring wraps twice and a
    half, and the compressed list grows to 80 rows): every step's output within 1e-2 of the
    oracle, whose window list is unbounded, and the row written at p lands at ring row p % 128.
    The ring's size does not depend on max_pos."""
    from smla import engine
    announce("decode layer window ring, 320 steps")
    t = _make_weights(4, seed=31)
    w = engine.LayerWeights(**{k: v.to(dev) for k, v in t.items()})
    wo = oe.OracleWeights(**{k: (v.double().numpy() if v.dtype == torch.bfloat16 else v.float())
                             for k, v in t.items()})
    B, max_pos, steps = 1, 512, 320
    layer = engine.DecodeLayer(w, B, 4, max_pos=max_pos, device=dev)
    assert tuple(layer.raw.shape) == (B, 128, 512)
    assert tuple(engine.DecodeLayer(w, B, 4, max_pos=4096, device=dev).raw.shape) == (B, 128, 512)
    st = oe.LayerState(4, max_pos=max_pos)
    g = torch.Generator().manual_seed(400)
    worst = 0.0
    for p in range(steps):
        xn = torch.randn(B, 4096, generator=g).to(torch.bfloat16)
        y = layer.step(xn.to(dev), torch.full((B,), p, dtype=torch.int32, device=dev)).float().cpu()
        yr, kv, ids, _ = oe.decode_step(st, wo, xn[0].float(), p)
        r = _rel(y[0], yr)
        worst = max(worst, r)
        assert r <= 1e-2, f"step {p}: output rel err {r:.3e}"
        _check_row(layer.raw[0, p % 128].float().cpu(), kv, 1e-2, f"step {p}: window row")
    announce(f"worst output rel err {worst:.3e}")


def test_prefill_rejects_bad_shapes(dev):
    from smla import engine
    t = _make_weights(0)
    layer = engine.DecodeLayer(engine.LayerWeights(**{k: v.to(dev) for k, v in t.items()}), 2, 0, max_pos=64,
                               device=dev)
    with pytest.raises(ValueError):
        layer.prefill(torch.zeros(2, 65, 4096, dtype=torch.bfloat16, device=dev))     # longer than max_pos
    with pytest.raises(ValueError):
        layer.prefill(torch.zeros(1, 8, 4096, dtype=torch.bfloat16, device=dev))      # wrong batch


def test_decode_layer_rejects_cpu_and_bad_ratio(dev):
    from smla import engine
    t = _make_weights(0)
    with pytest.raises(ValueError):
        engine.DecodeLayer(engine.LayerWeights(**{k: v.to(dev) for k, v in t.items()}), 1, ratio=2, max_pos=64,
                           device=dev)
    with pytest.raises(Exception):
        engine.DecodeLayer(engine.LayerWeights(**t), 1, ratio=0, max_pos=64, device=dev)   # CPU weights


def test_decode_layer_graph_replays(dev):
    """One decode step captured in a HIP graph and replayed token by token (new xn and pos copied
    into the captured inputs, eager work and synchronisations between replays) tracks an identical
    layer stepped eagerly, bit for bit, cache and ring state included."""
    from smla import engine
    announce("decode layer graph replays")
    t = _make_weights(4, seed=9)
    w = engine.LayerWeights(**{k: v.to(dev) for k, v in t.items()})
    B, max_pos = 2, 64
    eager = engine.DecodeLayer(w, B, 4, max_pos=max_pos, device=dev)
    graphed = engine.DecodeLayer(w, B, 4, max_pos=max_pos, device=dev)
    g = torch.Generator().manual_seed(3)
    xs = [torch.randn(B, 4096, generator=g).to(torch.bfloat16).to(dev) for _ in range(12)]
    # positions 0..3 eagerly on both, so the captured step starts from a warm state
    for p in range(4):
        pos = torch.full((B,), p, dtype=torch.int32, device=dev)
        eager.step(xs[p], pos)
        graphed.step(xs[p], pos)
    x_in = xs[4].clone()
    pos_in = torch.full((B,), 4, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_out = graphed.step(x_in, pos_in)
    # the capture itself ran nothing: step 4 is the first replay
    for p in range(4, 12):
        x_in.copy_(xs[p])
        pos_in.fill_(p)
        graph.replay()
        torch.cuda.synchronize()
        y_ref = eager.step(xs[p], torch.full((B,), p, dtype=torch.int32, device=dev))
        torch.cuda.synchronize()
        assert torch.equal(y_out, y_ref), f"replay at position {p}"
    assert torch.equal(graphed.raw, eager.raw) and torch.equal(graphed.comp32, eager.comp32)
