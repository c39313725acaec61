"""One sparse-MLA attention layer at decode, on the GPU: the caller-side wiring of
``oracle/decode_engine.py:73-119`` (``layer_fwd``'s decode branch, from the attention-normed input
``xn`` to ``o_grouped``; the hyper-connection mixing around it, ``hc_pre`` / ``hc_post``, belongs
to the model, not to this path).

``DecodeLayer.prefill`` ingests a prompt (the branch with ``decode_pos=None``, ``:86-95,107-117``);
``DecodeLayer.step`` then advances one token per call.  Per token at position p, for each of B
sequences:

* q  = perhead_norm(q_up(rmsnorm(q_down(xn), q_a_norm))), RoPE on the last 64 dims of each head
  (``decode_engine.py:78-80``);
* kv = rmsnorm(kv_proj(xn), kv_a_norm), RoPE on its last 64 dims, the fp8 round trip (e4m3,
  power-of-two scale per 64) on the other 448, written to row p % 128 of the 128-row window ring
  (``:81-84``, bounded as ``oracle/v4_fast.py:93-96`` keeps it: ``winr[p % 128]``);
* ratio-4 layers: the compressor ring takes xn @ wkv_c^T and xn @ wgate_c^T (+ ape) and emits a
  compressed row every 4 tokens (``:96-105``);
* ids: the ring rows of positions max(0, p-127)..p (position pp at row pp % 128, the ring order
  of ``ref_torch/sparse_attn.py:11-13``), then every causally visible compressed row, (p+1) // 4
  of them (``:110-114``, take-all); with indexer scores supplied, the window plus the top-k
  compressed rows instead;
* o = sparse_attn(q, [window; compressed], sinks, ids, 512^-0.5), the inverse RoPE on o's last
  64 dims, then ``o_grouped`` (``:115-119``).

RoPE tables: layers with a nonzero ratio (4 or 128) use YaRN (base 160000, factor 16 over 65536
positions), ratio-0 layers plain base 10000 (``decode_engine.py:47,73``).  Every step runs on the HIP kernels:
``smla_linear`` (projections, fp32 results), ``smla_row_epilogue`` (the norms, RoPE, the fp8 round
trip and the window-ring write; in a step, ``smla_ring_step_kv`` runs it with the compressor ring
step in one launch), ``smla_row_epilogue_ids`` (the per-head q epilogue with the id build),
``smla_select_decode`` (the indexer top-k form), ``smla_sparse_attn``, ``smla_prefill_attn``
(prompts) and ``smla_o_proj``.  Caches are device-resident and owned by the layer object: the
window is a 128-row ring whatever ``max_pos`` is, the compressed cache holds ``max_pos // 4``
rows (the reference's compressed list grows with the context the same way).
"""
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib, mla, ops
from . import compressor as _comp
from . import indexer as _idx
from . import norm_rope as _nr
from . import sparse_attn as _sa

HEAD_DIM, ROPE_HD, N_HEADS, WINDOW = 512, 64, 64, 128
_YARN = (65536, 160000.0, 16, 32, 1)   # original_seq_len, base, factor, beta_fast, beta_slow
_PLAIN = (0, 10000.0, 40, 32, 1)


@dataclass
class LayerWeights:
    """One layer's attention weights (bf16 on the GPU, norms and biases fp32), named as in the
    checkpoint (``blk.{L}.attn_*``): wq_a [1024, 4096], q_a_norm [1024], wq_b [64*512, 1024],
    wkv [512, 4096], kv_a_norm [512], wo_a [8*1024, 4096], wo_b [4096, 8192], sinks [64]; ratio-4
    layers add the compressor's wkv_c / wgate_c [1024, 4096], ape [4, 1024] and norm_c [512]."""
    wq_a: torch.Tensor
    q_a_norm: torch.Tensor
    wq_b: torch.Tensor
    wkv: torch.Tensor
    kv_a_norm: torch.Tensor
    wo_a: torch.Tensor
    wo_b: torch.Tensor
    sinks: torch.Tensor
    wkv_c: Optional[torch.Tensor] = None
    wgate_c: Optional[torch.Tensor] = None
    ape: Optional[torch.Tensor] = None
    norm_c: Optional[torch.Tensor] = None


def _proj(x, W):
    """x @ W^T with an fp32 result (bf16 operands, fp32 accumulation), ``smla_linear``."""
    return ops.linear_op(x.contiguous(), W, 1, torch.float32)


class DecodeLayer:
    """Decode state and step of one attention layer for B sequences.

    ``ratio`` is the layer's compression ratio (``decode_engine.py:17``): 4 runs the compressor ring
    and attends to the compressed rows; 0 and 128 attend to the window only (128 with the YaRN
    tables, as every nonzero ratio: ``oracle/v4_fast.py:42-43``).
    ``max_pos`` bounds the positions (the RoPE tables); the window is a ring of 128 rows and the
    compressed cache holds max_pos // 4 rows.  ``step`` advances every sequence by one token.
    """

    def __init__(self, w: LayerWeights, B: int, ratio: int, max_pos: int = 65536, device="cuda"):
        if ratio not in (0, 4, 128):
            raise ValueError("ratio must be 0, 4 or 128")
        if ratio == 4 and any(t is None for t in (w.wkv_c, w.wgate_c, w.ape, w.norm_c)):
            raise ValueError("a ratio-4 layer needs the compressor weights")
        ops._on_gpu(w.wq_a, w.wq_b, w.wkv, w.wo_a, w.wo_b)
        self.w, self.B, self.ratio, self.max_pos = w, B, ratio, max_pos
        self.cos_t, self.sin_t = _nr.rope_tables(ROPE_HD, max_pos, *(_YARN if ratio else _PLAIN), device=device)
        # the window ring: position p at row p % 128 (oracle/v4_fast.py:93-96)
        self.raw = torch.zeros(B, WINDOW, HEAD_DIM, dtype=torch.bfloat16, device=device)
        self.ring_ratio = 4 if ratio == 4 else 0  # only ratio-4 layers run the ring (decode_engine.py:86)
        self.ncap = max_pos // 4 if self.ring_ratio else 0
        if self.ring_ratio:
            self.comp32 = torch.zeros(B, self.ncap, HEAD_DIM, device=device)      # the ring writes fp32 rows
            self.comp = torch.zeros(B, self.ncap, HEAD_DIM, dtype=torch.bfloat16, device=device)
            self.ring = _comp.Ring(B, HEAD_DIM, w.ape, w.norm_c, ratio=4, rope_head_dim=ROPE_HD,
                                   max_pos=max_pos, fp8_sim=True, device=device, rope_args=_YARN)
        else:
            self.comp = torch.zeros(B, 1, HEAD_DIM, dtype=torch.bfloat16, device=device)   # never addressed
        self.q_a_norm = w.q_a_norm.float().contiguous()
        self.kv_a_norm = w.kv_a_norm.float().contiguous()
        # the projections of xn in one launch: [wq_a; wkv (; wkv_c; wgate_c)] concatenated once
        parts = [w.wq_a, w.wkv] + ([w.wkv_c, w.wgate_c] if self.ring_ratio else [])
        self.w_in = torch.cat(parts, dim=0).contiguous()
        self.cuts = [0]
        for t in parts:
            self.cuts.append(self.cuts[-1] + t.shape[0])

    # -- pieces (each mirrors one span of decode_engine.py) --------------------------------------
    def q_path(self, qa_f, pos):
        """``decode_engine.py:78-80``: q [rows, 64, 512] bf16 from the q_down projection qa_f
        [rows, 1024] of tokens at positions pos [rows], per-head normed, rope dims rotated."""
        rows = qa_f.shape[0]
        qa = torch.empty(rows, qa_f.shape[1], dtype=torch.bfloat16, device=qa_f.device)
        ops.row_epilogue(qa_f, self.q_a_norm, None, None, None, 0, _lib.SIM_NONE, qa)
        q = torch.empty(rows, N_HEADS, HEAD_DIM, dtype=torch.bfloat16, device=qa_f.device)
        ops.row_epilogue(_proj(qa, self.w.wq_b).view(rows * N_HEADS, HEAD_DIM), None, pos, self.cos_t, self.sin_t,
                         ROPE_HD, _lib.SIM_NONE, q, rows_per_pos=N_HEADS)
        return q

    def kv_append(self, kv_f, pos):
        """``decode_engine.py:81-84``: the token's kv row from the kv_proj projection kv_f
        (RMSNorm, RoPE of the last 64 dims, fp8 round trip of the other 448), written as bf16 to
        window-ring row pos % 128 of each sequence."""
        ops.row_epilogue(kv_f, self.kv_a_norm, pos, self.cos_t, self.sin_t, ROPE_HD, _lib.SIM_FP8, self.raw,
                         cache_rows=WINDOW)

    def ring_step(self, kvp, scp, pos):
        """``decode_engine.py:96-105``: ring update from the compressor projections; an emitted
        row lands in the fp32 compressed cache (its bf16 copy is made with the id list)."""
        self.ring.step(kvp, scp, pos, self.comp32)

    def index_list(self, pos, scores=None, k=2048):
        """``decode_engine.py:110-114``: [B, 128 + n] int32 ids into [window ring; compressed
        cache] (window ids are ring rows, compressed ids offset by 128), -1 padded.  Take-all over the visible compressed
        rows, or, with indexer scores [B, ncap] supplied, the top-k of the min((p+1)//4, ncap)
        visible ones (all of them, -1 padded, while at most k are visible).  Also copies a row the
        ring emitted at this step to the bf16 compressed cache."""
        comp = (self.comp32, self.comp) if self.ring_ratio else (None, None)
        take_all = scores is None or not self.ring_ratio
        T = WINDOW + (self.ncap if take_all else 0)
        ids = ops.decode_ids(pos, WINDOW, self.ring_ratio, WINDOW, self.ncap, T, comp32=comp[0],
                             comp_out=comp[1])
        if take_all:
            return ids
        return self._select(pos, scores, k)

    def q_and_ids(self, qa_f, pos, scores=None, k=2048):
        """``q_path`` and ``index_list`` of one decode step, with the per-head q epilogue and the id
        build in one launch (``smla_row_epilogue_ids``): the same q and ids.  Runs after the ring
        step, whose emitted row the id build copies."""
        rows = qa_f.shape[0]
        qa = torch.empty(rows, qa_f.shape[1], dtype=torch.bfloat16, device=qa_f.device)
        ops.row_epilogue(qa_f, self.q_a_norm, None, None, None, 0, _lib.SIM_NONE, qa)
        q = torch.empty(rows, N_HEADS, HEAD_DIM, dtype=torch.bfloat16, device=qa_f.device)
        comp = (self.comp32, self.comp) if self.ring_ratio else (None, None)
        take_all = scores is None or not self.ring_ratio
        T = WINDOW + (self.ncap if take_all else 0)
        # on the indexer-scores path this launch still builds the window ids (T = 128), because it
        # also makes the bf16 copy of a compressed row the ring emitted; _select then writes the
        # step's list (window + top-k) and those ids are not used
        ids = torch.empty(self.B, T, dtype=torch.int32, device=qa_f.device)
        ops.row_epilogue_ids(_proj(qa, self.w.wq_b).view(rows * N_HEADS, HEAD_DIM), None, pos, self.cos_t,
                             self.sin_t, ROPE_HD, _lib.SIM_NONE, q, N_HEADS, pos, WINDOW, self.ring_ratio,
                             WINDOW, self.ncap, T, ids, comp32=comp[0], comp_out=comp[1])
        if take_all:
            return q, ids
        return q, self._select(pos, scores, k)

    def _select(self, pos, scores, k):
        """Window + top-k ids from indexer scores [B, ncap] (``decode_engine.py:110-114``)."""
        if scores.shape != (self.B, self.ncap):
            raise ValueError(f"scores must be [{self.B}, {self.ncap}] (one per compressed slot)")
        # visible compressed rows at p: (p+1)//4 (decode_engine.py:112), at most the cache's rows
        nvis = torch.clamp(torch.div(pos + 1, 4, rounding_mode="floor"), max=self.ncap).to(torch.int32)
        return _idx.select_decode_indices(scores, k, pos, WINDOW, WINDOW, nvis=nvis)

    # -- prompt ingestion ------------------------------------------------------------------------
    def prefill(self, xn):
        """``decode_engine.py:73-117`` with ``decode_pos=None``: the prompt of every sequence, xn
        [B, S, 4096] bf16 at positions 0..S-1 (S <= max_pos), into a fresh layer.  Writes the S
        window rows into a transient prompt buffer; a ratio-4 layer pools the prompt's S // 4
        compressed rows (the gated pool of ``compressor_prefill`` with the fp8 round trip,
        ``:87-89``) and sets the ring from its last group and remainder (``:90-95``); then every
        position attends to its window and the compressed rows visible to it (``:107-116``), and
        the last min(S, 128) window rows go to their window-ring rows (``oracle/v4_fast.py:93-94``).
        Returns the layer's attention output [B, S, 4096] bf16; decoding continues with ``step``
        at position S."""
        ops._on_gpu(xn)
        if xn.dim() != 3 or xn.shape[0] != self.B or xn.shape[2] != self.w.wq_a.shape[1]:
            raise ValueError(f"xn must be [{self.B}, S, {self.w.wq_a.shape[1]}]")
        B, S, dim = xn.shape
        if not 0 < S <= self.max_pos:
            raise ValueError(f"the prompt length must lie in 1..{self.max_pos}")
        dev = xn.device
        pos = torch.arange(S, dtype=torch.int32, device=dev).repeat(B)      # position of each (b, s) row
        y = _proj(xn.reshape(B * S, dim), self.w_in)                        # [B*S, projection widths] fp32
        c = self.cuts
        q = self.q_path(y[:, c[0]:c[1]], pos)                               # [B*S, 64, 512]
        win = torch.empty(B, S, HEAD_DIM, dtype=torch.bfloat16, device=dev)    # the prompt's window rows
        for b in range(B):                                                  # window rows 0..S-1
            ops.row_epilogue(y[b * S:(b + 1) * S, c[1]:c[2]], self.kv_a_norm, pos[:S], self.cos_t, self.sin_t,
                             ROPE_HD, _lib.SIM_FP8, win[b])
        T = WINDOW
        if self.ring_ratio:
            kvp = y[:, c[2]:c[3]].reshape(B, S, -1)
            scp = y[:, c[3]:c[4]].reshape(B, S, -1)
            cut = S - S % 4
            if cut >= 4:
                comp = ops.gated_pool_op(kvp[:, :cut], scp[:, :cut], self.ring.ape, self.ring.norm_w, self.ring.cos_t,
                                         self.ring.sin_t, 4, ROPE_HD, 1e-6, _lib.SIM_FP8)
                self.comp32[:, :cut // 4] = comp
                self.comp[:, :cut // 4] = comp.to(torch.bfloat16)
            self.ring.init_from_prefill(kvp, scp)
            T += S // 4
        # every position's window and visible compressed rows, computed in the kernel (smla_prefill_attn)
        o = _sa.prefill_attn(q.view(B, S, N_HEADS, HEAD_DIM), win, self.comp if self.ring_ratio else None,
                             self.w.sinks.float(), HEAD_DIM ** -0.5, q_pos0=0, window=WINDOW, ratio=self.ring_ratio,
                             dv=HEAD_DIM)
        lo = max(0, S - WINDOW)                     # the positions the ring keeps, each at its row p % 128
        self.raw[:, torch.arange(lo, S, device=dev) % WINDOW] = win[:, lo:]
        out = mla.o_project(o.view(B * S, N_HEADS, HEAD_DIM), pos, self.cos_t, self.sin_t, self.w.wo_a, self.w.wo_b)
        return out.view(B, S, -1)

    # -- the step --------------------------------------------------------------------------------
    def step(self, xn, pos, scores=None, k=2048):
        """xn [B, 4096] bf16 (the attention-normed input), pos [B] int32 on the GPU, the same
        position sequence for every call of a sequence (p, p+1, ...), each in [0, max_pos).
        Returns the layer's attention output [B, 4096] bf16 (``o_grouped``'s result, before
        ``hc_post``).  Outside graph capture the positions are checked against max_pos (one
        device read); a captured step relies on the caller's positions."""
        ops._on_gpu(xn, pos)
        if xn.shape != (self.B, self.w.wq_a.shape[1]):
            raise ValueError(f"xn must be [{self.B}, {self.w.wq_a.shape[1]}]")
        if pos.shape != (self.B,):
            raise ValueError(f"pos must be [{self.B}]")
        pos = pos.to(torch.int32).contiguous()
        if not torch.cuda.is_current_stream_capturing():
            lo, hi = torch.aminmax(pos)
            if int(lo) < 0 or int(hi) >= self.max_pos:
                raise ValueError(f"positions must lie in [0, {self.max_pos}); got {int(lo)}..{int(hi)}")
        y = _proj(xn, self.w_in)                     # [B, sum of the projection widths] fp32
        c = self.cuts
        if self.ring_ratio:
            # the kv row's epilogue and the ring step in one launch (kv_append + ring_step)
            ops.ring_step_kv(self.ring, y[:, c[2]:c[3]], y[:, c[3]:c[4]], pos, self.comp32, y[:, c[1]:c[2]],
                             self.kv_a_norm, self.cos_t, self.sin_t, ROPE_HD, _lib.SIM_FP8, self.raw,
                             cache_rows=WINDOW)
        else:
            self.kv_append(y[:, c[1]:c[2]], pos)
        q, ids = self.q_and_ids(y[:, c[0]:c[1]], pos, scores, k)
        o = _sa.sparse_attn_two_source(q[:, None], self.raw, self.comp, self.w.sinks.float(), ids[:, None],
                                       HEAD_DIM ** -0.5, dv=HEAD_DIM)
        return mla.o_project(o[:, 0].contiguous(), pos, self.cos_t, self.sin_t, self.w.wo_a, self.w.wo_b)
