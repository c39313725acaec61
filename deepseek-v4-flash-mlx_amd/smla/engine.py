"""One sparse-MLA attention layer at decode, on the GPU: the caller-side wiring of
``oracle/decode_engine.py:73-119`` (``layer_fwd``'s decode branch, from the attention-normed input
``xn`` to ``o_grouped``; the hyper-connection mixing around it, ``hc_pre`` / ``hc_post``, belongs
to the model, not to this path).

Per token at position p, for each of B sequences:

* q  = perhead_norm(q_up(rmsnorm(q_down(xn), q_a_norm))), RoPE on the last 64 dims of each head
  (``decode_engine.py:78-80``);
* kv = rmsnorm(kv_proj(xn), kv_a_norm), RoPE on its last 64 dims, the fp8 round trip (e4m3,
  power-of-two scale per 64) on the other 448, written to window-cache row p (``:81-84``);
* ratio-4 layers: the compressor ring takes xn @ wkv_c^T and xn @ wgate_c^T (+ ape) and emits a
  compressed row every 4 tokens (``:96-105``);
* ids: window rows max(0, p-127)..p, then every causally visible compressed row, (p+1) // 4 of
  them (``:110-114``, take-all); with indexer scores supplied, the window plus the top-k
  compressed rows instead;
* o = sparse_attn(q, [window; compressed], sinks, ids, 512^-0.5), the inverse RoPE on o's last
  64 dims, then ``o_grouped`` (``:115-119``).

RoPE tables: ratio-4 layers use YaRN (base 160000, factor 16 over 65536 positions), ratio-0
layers plain base 10000 (``decode_engine.py:47,73``).  Every step runs on the HIP kernels:
``smla_linear`` (projections, fp32 results), ``smla_rope``, ``smla_quant_fp8_pow2``, ``smla_ring_step``,
``smla_sparse_attn`` and ``smla_o_proj``; the norms and the index build are torch element-wise
work on the GPU.  Caches are device-resident and owned by the layer object.
"""
from dataclasses import dataclass
from typing import Optional

import torch

from . import mla, ops
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
    """x @ W^T with an fp32 result: the HIP projection kernel at decode shapes (bf16 operands, fp32
    accumulation and output), a float32 product otherwise."""
    if mla._decode_shape(x, W) and W.shape[0] % 16 == 0:
        return ops.linear_op(x.contiguous(), W, 1, torch.float32)
    return x.float() @ W.float().t()


def _e4m3_table(device):
    """fp32 value of each of the 256 e4m3 codes (the two NaN codes never occur: the quantiser
    clamps to +-448)."""
    return torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().to(device)


class DecodeLayer:
    """Decode state and step of one attention layer for B sequences.

    ``ratio`` is the layer's compression ratio (4: compressed rows and the ring; 0: window only).
    ``max_pos`` bounds the positions (window cache rows); the compressed cache holds
    max_pos // 4 rows.  ``step`` advances every sequence by one token.
    """

    def __init__(self, w: LayerWeights, B: int, ratio: int, max_pos: int = 65536, device="cuda"):
        if ratio not in (0, 4):
            raise ValueError("ratio must be 0 or 4")
        if ratio == 4 and any(t is None for t in (w.wkv_c, w.wgate_c, w.ape, w.norm_c)):
            raise ValueError("a ratio-4 layer needs the compressor weights")
        ops._on_gpu(w.wq_a, w.wq_b, w.wkv, w.wo_a, w.wo_b)
        self.w, self.B, self.ratio, self.max_pos = w, B, ratio, max_pos
        self.cos_t, self.sin_t = _nr.rope_tables(ROPE_HD, max_pos, *(_YARN if ratio else _PLAIN), device=device)
        self.raw = torch.zeros(B, max_pos, HEAD_DIM, dtype=torch.bfloat16, device=device)
        self.ncap = max_pos // 4 if ratio else 0
        if ratio:
            self.comp32 = torch.zeros(B, self.ncap, HEAD_DIM, device=device)      # the ring writes fp32 rows
            self.comp = torch.zeros(B, self.ncap, HEAD_DIM, dtype=torch.bfloat16, device=device)
            self.ring = _comp.Ring(B, HEAD_DIM, w.ape, w.norm_c, ratio=4, rope_head_dim=ROPE_HD,
                                   max_pos=max_pos, fp8_sim=True, device=device, rope_args=_YARN)
        else:
            self.comp = torch.zeros(B, 1, HEAD_DIM, dtype=torch.bfloat16, device=device)   # never addressed
        self.e4m3 = _e4m3_table(device)
        self.rows = torch.arange(B, device=device)

    # -- pieces (each mirrors one span of decode_engine.py) --------------------------------------
    def q_path(self, xn, pos):
        """``decode_engine.py:78-80``: q [B, 64, 512] bf16 with its rope dims rotated."""
        w = self.w
        qa = _nr.rmsnorm(_proj(xn, w.wq_a), w.q_a_norm).to(torch.bfloat16)
        q = _proj(qa, w.wq_b).reshape(self.B, N_HEADS, HEAD_DIM)
        q = mla.perhead_norm(q).to(torch.bfloat16).contiguous()
        ops.rope_op_(q, pos, self.cos_t, self.sin_t, False)
        return q

    def kv_row(self, xn, pos):
        """``decode_engine.py:81-83``: the token's window row [B, 512] fp32 (RoPE on the last 64
        dims, fp8 round trip on the other 448)."""
        w = self.w
        kv = _nr.rmsnorm(_proj(xn, w.wkv), w.kv_a_norm).contiguous()   # fp32 from here on
        ops.rope_op_(kv[:, None, :], pos, self.cos_t, self.sin_t, False)
        nope = kv[:, :HEAD_DIM - ROPE_HD].contiguous()
        codes, scales = ops.quant_fp8_pow2_op(nope)
        kv[:, :HEAD_DIM - ROPE_HD] = self.e4m3[codes.long()] * scales.repeat_interleave(64, dim=-1)
        return kv

    def ring_step(self, xn, pos):
        """``decode_engine.py:96-105``: ring update; an emitted row lands in the compressed cache."""
        w = self.w
        kvp = _proj(xn, w.wkv_c)
        scp = _proj(xn, w.wgate_c)
        self.ring.step(kvp, scp, pos, self.comp32)
        emitted = (pos + 1) % 4 == 0
        r = ((pos + 1) // 4 - 1).clamp(min=0).long()
        cur = self.comp[self.rows, r]
        self.comp[self.rows, r] = torch.where(emitted[:, None], self.comp32[self.rows, r].to(torch.bfloat16), cur)

    def index_list(self, pos, scores=None, k=2048):
        """``decode_engine.py:110-114``: [B, 128 + n] int32 ids into [window cache; compressed
        cache] (compressed ids offset by max_pos), -1 padded.  Take-all over the visible compressed
        rows, or, with indexer scores [B, ncap] supplied, the top-k of them."""
        if scores is not None and self.ratio:
            return _idx.select_decode_indices(scores, k, pos, WINDOW, self.max_pos)
        p = pos.long()[:, None]
        j = torch.arange(WINDOW, device=pos.device)[None]
        lo = (p - (WINDOW - 1)).clamp(min=0)
        wid = lo + j
        wid = torch.where(wid <= p, wid, torch.full_like(wid, -1))
        if not self.ratio:
            return wid.to(torch.int32)
        c = torch.arange(self.ncap, device=pos.device)[None]
        cid = torch.where(c < (p + 1) // 4, self.max_pos + c, torch.full_like(c, -1))
        return torch.cat([wid, cid], dim=1).to(torch.int32)

    # -- the step --------------------------------------------------------------------------------
    def step(self, xn, pos, scores=None, k=2048):
        """xn [B, 4096] bf16 (the attention-normed input), pos [B] int32 on the GPU, the same
        position sequence for every call of a sequence (p, p+1, ...).  Returns the layer's
        attention output [B, 4096] bf16 (``o_grouped``'s result, before ``hc_post``)."""
        ops._on_gpu(xn, pos)
        if xn.shape != (self.B, self.w.wq_a.shape[1]):
            raise ValueError(f"xn must be [{self.B}, {self.w.wq_a.shape[1]}]")
        pos = pos.to(torch.int32).contiguous()
        q = self.q_path(xn, pos)
        kv = self.kv_row(xn, pos)
        self.raw[self.rows, pos.long()] = kv.to(torch.bfloat16)
        if self.ratio:
            self.ring_step(xn, pos)
        ids = self.index_list(pos, scores, k)
        o = _sa.sparse_attn_two_source(q[:, None], self.raw, self.comp, self.w.sinks.float(), ids[:, None],
                                       HEAD_DIM ** -0.5, dv=HEAD_DIM)
        return mla.o_project(o[:, 0].contiguous(), pos, self.cos_t, self.sin_t, self.w.wo_a, self.w.wo_b)
