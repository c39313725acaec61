"""Decode step of one sparse-MLA attention layer (CPU oracle; test infrastructure only).

Restates ``oracle/decode_engine.py:73-119`` (``layer_fwd``'s decode branch for one token at
position p, from the attention-normed input xn to ``o_grouped``; ``hc_pre`` / ``hc_post`` are
outside the path), composed from the oracle's own pieces:

* RoPE tables by layer ratio (``:47,73``): a nonzero ratio (4 or 128) -> YaRN (original 65536,
  base 160000, factor 16, beta 32/1), ratio 0 -> plain base 10000 (original_seq_len 0); only
  ratio-4 layers run the compressor and see compressed rows (``:86,112``);
* q (``:78-80``): q_down, RMSNorm(q_a_norm), q_up to [64, 512], the weightless per-head RMS norm
  (``v4mlx/mla.py:26-28``), RoPE at p on each head's last 64 dims;
* kv (``:81-84``): kv_proj, RMSNorm(kv_a_norm), RoPE at p on the last 64 dims, the fp8 round
  trip on the first 448 (``fp8.act_quant_sim``), appended to the window list;
* ratio-4 layers (``:96-105``): ``compressor.ring_step`` with the projections x @ wkv_c^T,
  x @ wgate_c^T and the YaRN frequencies of ``decode_engine.py:48``; an emitted row is appended
  to the compressed list;
* attention (``:107-116``): kv buffer [window list; compressed list], ids = positions
  max(0, p-127)..p, then the first min(n_comp, (p+1)//4) compressed rows; ``sparse_attn`` with
  the sinks and scale 512^-0.5;
* output (``:118-119``): ``mla.o_project`` (inverse RoPE at p, then ``o_grouped``).

Products run in float64 (``mla.linear``), norms and rotations in float32 as the pieces define.

Pinning (``tests/test_oracle_engine.py``): the emission schedule (one compressed row after every
4th token, none for ratio 0), the id lists against a brute-force enumeration, the first step's
attention against the one-row closed form o = v e^s / (e^s + e^sink), and the window row's
rotation against the rotation at position p applied to the unrotated row (a wrong position or a
dropped RoPE fails it).
"""
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import compressor as _comp
from . import fp8 as _fp8
from . import indexer as _idx
from . import mla as _mla
from . import norm_rope as _nr
from . import sparse_attn as _sa

RD, WINDOW = 64, 128
YARN = (65536, 160000.0, 16, 32, 1)
PLAIN = (0, 10000.0, 40, 32, 1)


@dataclass
class OracleWeights:
    """fp32 / float64 copies of one layer's attention weights (same names as the checkpoint's
    ``blk.{L}.attn_*``)."""
    wq_a: np.ndarray
    q_a_norm: torch.Tensor
    wq_b: np.ndarray
    wkv: np.ndarray
    kv_a_norm: torch.Tensor
    wo_a: np.ndarray
    wo_b: np.ndarray
    sinks: torch.Tensor
    wkv_c: Optional[np.ndarray] = None
    wgate_c: Optional[np.ndarray] = None
    ape: Optional[torch.Tensor] = None
    norm_c: Optional[torch.Tensor] = None


class LayerState:
    """``oracle/decode_engine.py:68-69``: the window list, the compressed list and the ring."""

    def __init__(self, ratio, max_pos=65536):
        self.ratio = ratio
        self.win, self.comp = [], []
        self.kvs = torch.zeros(2 * 4, 2 * 512)
        self.scs = torch.full((2 * 4, 2 * 512), float("-inf"))
        self.cos, self.sin = _nr.rope_cos_sin(RD, max_pos, *(YARN if ratio else PLAIN))
        self.freqs_c = _nr.precompute_freqs(RD, 64, *YARN)


def rope_at(x, st, p, inverse=False):
    """Rotate the interleaved pairs of x [..., 64] (fp32) to position p with the layer's table."""
    cis = torch.complex(st.cos[p:p + 1], st.sin[p:p + 1])                 # [1, 32]
    lead = x.shape[:-1]
    y = _nr.apply_rotary_emb(x.reshape(1, 1, -1, RD), cis, inverse=inverse)
    return y.reshape(*lead, RD)


def index_list(p, n_window_rows, n_comp, ratio, scores=None, k=2048):
    """``oracle/decode_engine.py:110-114`` over [window list (one row per position from 0);
    compressed list].  With indexer scores (one per compressed slot), the compressed ids are the
    top-k of the min(n_comp, (p+1)//4) visible slots by (score desc, index asc), ascending
    (``indexer.topk``), in place of all of them."""
    widx = list(range(max(0, p - WINDOW + 1), p + 1))
    nvis = min(n_comp, (p + 1) // 4) if ratio == 4 else 0
    if scores is None or ratio != 4:
        cidx = [n_window_rows + j for j in range(nvis)]
    else:
        sel = _idx.topk(np.asarray(scores, dtype=np.float32)[None], k, nvis=np.array([nvis], dtype=np.int32))[0]
        cidx = [n_window_rows + int(j) for j in sel if j >= 0]
    return torch.tensor(widx + cidx, dtype=torch.int32)


def prefill(st, w, xn):
    """The prefill branch of ``oracle/decode_engine.py:73-117`` for a prompt at positions 0..S-1:
    xn [S, dim] (fp32).  Appends every token's window row, fills the compressed list with the
    prompt's pooled rows (``compressor.gated_pool`` over the float64 projections, then the fp8
    round trip of the non-rope dims, ``:87-89``) and sets the ring from the prompt's last group
    (``compressor.ring_init``, ``:90-95``); then each position i attends to window rows
    max(0, i-127)..i and the first min(n_comp, (i+1)//4) compressed rows of the whole prompt's
    [window; compressed] buffer (``:107-116``).  Returns (y [S, dim_out] float64, ids per position,
    o [S, 64, 512] fp32)."""
    x = np.asarray(xn, dtype=np.float64)
    S = x.shape[0]
    qa = _nr.rmsnorm(torch.from_numpy(_mla.linear(x, w.wq_a)).float(), w.q_a_norm)
    q = torch.from_numpy(_mla.linear(qa.numpy(), w.wq_b)).float().reshape(S, 64, 512)
    q = q * torch.rsqrt(q.pow(2).mean(-1, keepdim=True) + 1e-6)
    q = torch.stack([torch.cat([q[i, :, :-RD], rope_at(q[i, :, -RD:], st, i)], dim=-1) for i in range(S)])
    kvn = _nr.rmsnorm(torch.from_numpy(_mla.linear(x, w.wkv)).float(), w.kv_a_norm)
    for i in range(S):
        kv = torch.cat([kvn[i, :-RD], rope_at(kvn[i, -RD:], st, i)])
        nope, _ = _fp8.act_quant_sim(kv[:-RD].numpy()[None], 64)
        st.win.append(torch.cat([torch.from_numpy(nope[0]), kv[-RD:]]))
    if st.ratio == 4:
        kvf = torch.from_numpy(_mla.linear(x, w.wkv_c)).float()
        scf = torch.from_numpy(_mla.linear(x, w.wgate_c)).float()
        cut = S - S % 4
        if cut >= 4:
            freqs = _nr.precompute_freqs_cis(RD, S, *YARN)
            comp = _comp.gated_pool(kvf[None, :cut], scf[None, :cut], w.ape, w.norm_c, freqs, 4, RD)[0]
            nope, _ = _fp8.act_quant_sim(comp[:, :-RD].numpy(), 64)
            comp = torch.cat([torch.from_numpy(nope), comp[:, -RD:]], dim=-1)
            st.comp = [comp[j] for j in range(comp.shape[0])]
        st.kvs, st.scs = _comp.ring_init(kvf, scf, w.ape, 4)
    kvcat = torch.stack(st.win + st.comp)
    ids_all, o_all = [], []
    for i in range(S):
        ids = index_list(i, len(st.win), len(st.comp), st.ratio)
        ids_all.append(ids)
        o_all.append(_sa.sparse_attn(q[i][None], kvcat, w.sinks, ids[None], 512 ** -0.5)[0])
    o = torch.stack(o_all)
    y = _mla.o_project(o, torch.arange(S), st.cos, st.sin, w.wo_a, w.wo_b)
    return np.asarray(y), ids_all, o


def decode_step(st, w, xn, p, scores=None, k=2048):
    """One token at position p: xn [dim] (fp32); optional indexer scores [n_slots] select the
    top-k visible compressed rows (``index_list``).  Returns (y [dim_out] float64, the window row
    [512] fp32, ids int32, o [64, 512] fp32 before the output projection)."""
    x = np.asarray(xn, dtype=np.float64)[None]
    qa = _nr.rmsnorm(torch.from_numpy(_mla.linear(x, w.wq_a)).float(), w.q_a_norm)
    q = torch.from_numpy(_mla.linear(qa.numpy(), w.wq_b)).float().reshape(64, 512)
    q = q * torch.rsqrt(q.pow(2).mean(-1, keepdim=True) + 1e-6)
    q = torch.cat([q[:, :-RD], rope_at(q[:, -RD:], st, p)], dim=-1)
    kv = _nr.rmsnorm(torch.from_numpy(_mla.linear(x, w.wkv)).float(), w.kv_a_norm)[0]
    kv = torch.cat([kv[:-RD], rope_at(kv[-RD:], st, p)])
    nope, _ = _fp8.act_quant_sim(kv[:-RD].numpy()[None], 64)
    kv = torch.cat([torch.from_numpy(nope[0]), kv[-RD:]])
    st.win.append(kv)
    if st.ratio == 4:
        kvp = torch.from_numpy(_mla.linear(x, w.wkv_c)).float()[0]
        scp = torch.from_numpy(_mla.linear(x, w.wgate_c)).float()[0]
        row = _comp.ring_step(st.kvs, st.scs, kvp, scp, p, w.ape, w.norm_c, st.freqs_c, 4, RD, fp8_sim=True)
        if row is not None:
            st.comp.append(row)
    ids = index_list(p, len(st.win), len(st.comp), st.ratio, scores, k)
    kvcat = torch.stack(st.win + st.comp)
    o = _sa.sparse_attn(q[None], kvcat, w.sinks, ids[None], 512 ** -0.5)          # [1, 64, 512]
    y = _mla.o_project(o, torch.tensor([p]), st.cos, st.sin, w.wo_a, w.wo_b)
    return np.asarray(y)[0], kv, ids, o[0]
