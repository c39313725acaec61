"""Pins the oracle's decode-layer composition (``oracle/engine.py``, restating
``oracle/decode_engine.py:73-119``) on small hidden sizes: the compressor's emission schedule, the
id lists against a brute-force enumeration, the first step's attention against the one-row closed
form, and the window row's rotation against the position-p rotation of the unrotated row."""
import math

import numpy as np
import pytest
import torch

from oracle import engine as oe
from oracle import fp8 as ofp8
from oracle import mla as omla
from oracle import norm_rope as onr


def _weights(seed, dim=256, q_lora=128, rank=32, dim_out=192, ratio=4):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, sc=0.05: (torch.randn(*s, generator=g) * sc)
    w = oe.OracleWeights(
        wq_a=r(q_lora, dim).numpy().astype(np.float64), q_a_norm=1 + r(q_lora, sc=0.1),
        wq_b=r(64 * 512, q_lora).numpy().astype(np.float64), wkv=r(512, dim).numpy().astype(np.float64),
        kv_a_norm=1 + r(512, sc=0.1), wo_a=r(8 * rank, 4096).numpy().astype(np.float64),
        wo_b=r(dim_out, 8 * rank).numpy().astype(np.float64), sinks=r(64, sc=1.0))
    if ratio == 4:
        w.wkv_c = r(1024, dim).numpy().astype(np.float64)
        w.wgate_c = r(1024, dim).numpy().astype(np.float64)
        w.ape = r(4, 1024, sc=0.1)
        w.norm_c = 1 + r(512, sc=0.1)
    return w, g


@pytest.mark.parametrize("ratio", [4, 0, 128])
def test_schedule_and_ids(ratio):
    w, g = _weights(1, ratio=ratio)
    st = oe.LayerState(ratio, max_pos=512)
    for p in range(11):
        _, _, ids, _ = oe.decode_step(st, w, torch.randn(256, generator=g), p)
        assert len(st.win) == p + 1
        assert len(st.comp) == ((p + 1) // 4 if ratio == 4 else 0)
        brute = [t for t in range(p + 1) if p - t < 128]
        brute += [len(st.win) + j for j in range(len(st.comp)) if j < (p + 1) // 4] if ratio == 4 else []
        assert ids.tolist() == brute


def test_window_slides_past_128():
    # the id rule alone, at positions beyond the window (no state needed)
    for p in (127, 128, 200):
        ids = oe.index_list(p, p + 1, (p + 1) // 4, 4).tolist()
        assert ids[:128] == list(range(p - 127, p + 1))
        assert ids[128:] == [p + 1 + j for j in range((p + 1) // 4)]


def test_first_step_closed_form():
    """At p = 0 the only row is the token's own window row v: o_h = v e^{s_h} / (e^{s_h} + e^{sink_h})
    with s_h = q_h . v / sqrt(512)."""
    w, g = _weights(2, ratio=0)
    st = oe.LayerState(0, max_pos=64)
    x = torch.randn(256, generator=g)
    _, v, ids, o = oe.decode_step(st, w, x, 0)
    assert ids.tolist() == [0]
    # q of the step, rebuilt from the pieces (position 0: cos 1, sin 0, so no rotation)
    qa = onr.rmsnorm(torch.from_numpy(omla.linear(x.numpy()[None], w.wq_a)).float(), w.q_a_norm)
    q = torch.from_numpy(omla.linear(qa.numpy(), w.wq_b)).float().reshape(64, 512)
    q = q * torch.rsqrt(q.pow(2).mean(-1, keepdim=True) + 1e-6)
    s = (q.double() @ v.double()) / math.sqrt(512)
    wgt = torch.exp(s) / (torch.exp(s) + torch.exp(w.sinks.double()))
    ref = wgt[:, None] * v.double()[None]
    assert torch.allclose(o.double(), ref, rtol=1e-4, atol=1e-6)


def test_window_row_rotated_at_its_position():
    """The window row's rope dims are the unrotated row's pairs turned by the angle of position p
    (x0 cos - x1 sin, x0 sin + x1 cos); the fp8 round trip covers exactly the other 448 dims."""
    w, g = _weights(3, ratio=0)
    st = oe.LayerState(0, max_pos=64)
    for p in range(6):
        x = torch.randn(256, generator=g)
        _, v, _, _ = oe.decode_step(st, w, x, p)
        kv = onr.rmsnorm(torch.from_numpy(omla.linear(x.numpy()[None], w.wkv)).float(), w.kv_a_norm)[0]
        a, b = kv[-64::2].double(), kv[-63::2].double()
        c, s = st.cos[p].double(), st.sin[p].double()
        rot = torch.stack([a * c - b * s, a * s + b * c], dim=-1).reshape(64)
        assert torch.allclose(v[-64:].double(), rot, rtol=1e-5, atol=1e-6)
        nope, _ = ofp8.act_quant_sim(kv[:-64].numpy()[None], 64)
        assert np.array_equal(v[:-64].numpy(), nope[0])
        if p > 0:  # a rotation at another position would not match
            c0, s0 = st.cos[p - 1].double(), st.sin[p - 1].double()
            wrong = torch.stack([a * c0 - b * s0, a * s0 + b * c0], dim=-1).reshape(64)
            assert not torch.allclose(v[-64:].double(), wrong, rtol=1e-3, atol=1e-4)


def test_rope_tables_by_ratio():
    """decode_engine.py:47,73: every nonzero ratio (4 and 128) rotates with the YaRN tables, ratio 0
    with the plain base-10000 ones; the two differ."""
    yc, _ = onr.rope_cos_sin(64, 256, *oe.YARN)
    pc, _ = onr.rope_cos_sin(64, 256, *oe.PLAIN)
    assert not torch.allclose(yc, pc)
    for ratio, ref in ((4, yc), (128, yc), (0, pc)):
        assert torch.equal(oe.LayerState(ratio, max_pos=256).cos, ref)


@pytest.mark.parametrize("ratio,S", [(4, 23), (0, 9), (4, 8)])
def test_prefill_equals_decode_steps(ratio, S):
    """The oracle prefill (the reference's prompt branch: every window row, the prompt's pooled
    compressed rows, the ring from its last group) against S decode steps from an empty state,
    which are pinned above: identical window rows and id lists, compressed rows and outputs equal
    to float32 rounding (pooling the whole prompt and stepping the ring order the same sums
    differently; the fp8 round trip may move a value by one e4m3 step), the same ring contents,
    and the same output at the next decode step."""
    w, g = _weights(5, ratio=ratio)
    xs = torch.randn(S + 1, 256, generator=g)
    a, b = oe.LayerState(ratio, max_pos=512), oe.LayerState(ratio, max_pos=512)
    y_pre, ids_pre, _ = oe.prefill(a, w, xs[:S])
    y_dec = []
    for p in range(S):
        y, _, ids, _ = oe.decode_step(b, w, xs[p], p)
        y_dec.append(y)
        # the id rule is positional; the compressed offset is the window length (S vs p + 1)
        want = [t for t in ids.tolist() if t <= p] + [S + (t - p - 1) for t in ids.tolist() if t > p]
        assert ids_pre[p].tolist() == want
    assert len(a.win) == len(b.win) == S
    for p in range(S):
        assert torch.equal(a.win[p], b.win[p])
    assert len(a.comp) == len(b.comp)
    for j in range(len(a.comp)):
        ra, rb = a.comp[j].numpy(), b.comp[j].numpy()
        np.testing.assert_allclose(ra[-64:], rb[-64:], rtol=1e-4, atol=1e-6)
        step = np.abs(rb[:-64]) * 2.0 ** -3 + 1e-6
        assert np.all(np.abs(ra[:-64] - rb[:-64]) <= step)
    np.testing.assert_allclose(y_pre, np.stack(y_dec), rtol=1e-3, atol=1e-3 * np.abs(y_pre).max())
    if ratio == 4:
        live = 4 + S % 4
        assert torch.equal(a.kvs[:live], b.kvs[:live]) and torch.equal(a.scs[:live], b.scs[:live])
    ya, _, _, _ = oe.decode_step(a, w, xs[S], S)
    yb, _, _, _ = oe.decode_step(b, w, xs[S], S)
    np.testing.assert_allclose(ya, yb, rtol=1e-3, atol=1e-3 * np.abs(yb).max())
