"""KV time-axis compressor: gated overlapped pooling, decode ring step, block mean pool (CPU oracle).

Restates:

* ``overlap_transform``  — ``ref_torch/compressor.py:12-18``: [b,g,r,2d] -> [b,g,2r,d]; slots
  r..2r-1 take the group's own second-half channels, slots 0..r-1 the previous group's
  first-half channels, group 0's first r slots take ``value``;
* ``compressor_prefill`` — ``ref_torch/compressor.py:21-50``: kv/score projections, per-slot
  bias ``ape`` on the scores, overlapped windows, per-channel softmax over the 2r slots,
  weighted sum, RMSNorm, RoPE of the last ``rope_head_dim`` channels at positions 0, r, 2r, ...
  It also returns the reference's state dict (last full group's kv and biased score, and the
  unpooled remainder kv);
* ``gated_pool``         — the same pooling starting from the projections (what the HIP kernel
  computes; the projections are an upstream GEMM);
* ``ring_step``          — the decode-time incremental compressor of
  ``oracle/decode_engine.py:96-105``: an 8-slot ring of (kv, biased score); every ``ratio``-th
  token the ring emits one row (softmax pooling, RMSNorm, RoPE at the group's first position,
  optional fp8 round trip of the non-rope channels) and shifts;
* ``mean_pool``          — plain block mean (r rows -> 1) used by the 32K decode workload,
  summed in row order and multiplied by 1/r in fp32.

Pinning: golden vectors from the reference for ``overlap_transform`` and ``compressor_prefill``
(outputs and state, ``tests/golden/``), the special cases "uniform scores => mean over the valid
slots" and "group 0 => softmax over its own r slots", a brute-force per-(group, channel) loop,
ring-vs-prefill equality (running the ring over a sequence reproduces the prefill rows), and the
closed form of ``mean_pool``.
"""
import torch

from . import fp8 as _fp8
from .norm_rope import apply_rotary_emb, precompute_freqs_cis, rmsnorm


def overlap_transform(tensor, ratio, d, value):
    """tensor:[b,g,ratio,2d] -> [b,g,2*ratio,d] (see module docstring)."""
    b, g = tensor.shape[0], tensor.shape[1]
    out = torch.full((b, g, 2 * ratio, d), value, dtype=tensor.dtype)
    out[:, :, ratio:, :] = tensor[..., d:]
    if g > 1:
        out[:, 1:, :ratio, :] = tensor[:, : g - 1, :, :d]
    return out


def _pool(kv, score, ratio, d):
    """Softmax-weighted sum over the overlapped 2*ratio slots. kv/score: [b, g*ratio, 2d]."""
    b, n, _ = kv.shape
    g = n // ratio
    kvo = overlap_transform(kv.reshape(b, g, ratio, 2 * d), ratio, d, 0.0)
    sco = overlap_transform(score.reshape(b, g, ratio, 2 * d), ratio, d, float("-inf"))
    wts = torch.softmax(sco, dim=2)
    return (kvo * wts).sum(dim=2)                                     # [b, g, d]


def gated_pool(kv, score, ape, norm_w, freqs_cis, ratio=4, rope_head_dim=64, eps=1e-6):
    """Pooling from projections. kv/score:[b, n, 2d] fp32 (n a multiple of ratio; remainder
    rows dropped), ape:[ratio, 2d], norm_w:[d], freqs_cis:[>= n, rd/2] complex -> [b, n//ratio, d].
    """
    b, n, two_d = kv.shape
    d = two_d // 2
    cut = n - n % ratio
    kv = kv[:, :cut].float()
    sc = (score[:, :cut].float().reshape(b, cut // ratio, ratio, two_d) + ape.float()).reshape(b, cut, two_d)
    pooled = _pool(kv, sc, ratio, d)
    pooled = rmsnorm(pooled, norm_w.float(), eps)
    rd = rope_head_dim
    rot = apply_rotary_emb(pooled[..., d - rd:], freqs_cis[:cut:ratio])
    return torch.cat([pooled[..., : d - rd], rot], dim=-1)


def compressor_prefill(x, wkv, wgate, ape, norm_w, head_dim=512, ratio=4, rope_head_dim=64,
                       base=160000.0, original_seq_len=65536, factor=16, beta_fast=32, beta_slow=1):
    """x:[b,s,dim] -> (kv:[b, s//ratio, head_dim] fp32 post-RoPE, state dict)."""
    b, s, _ = x.shape
    xf = x.float()
    kv = xf @ wkv.float().t()
    score = xf @ wgate.float().t()
    rem = s % ratio
    cut = s - rem
    state = {}
    if cut >= ratio:
        state["kv"] = kv[:, cut - ratio:cut].clone()
        state["score"] = (score[:, cut - ratio:cut] + ape.float()).clone()
    if rem > 0:
        state["kv_rem"] = kv[:, cut:].clone()
    freqs = precompute_freqs_cis(rope_head_dim, s, original_seq_len, base, factor, beta_fast, beta_slow)
    out = gated_pool(kv[:, :cut], score[:, :cut], ape, norm_w, freqs, ratio, rope_head_dim)
    return out, state


def ring_init(kv_proj, score_proj, ape, ratio=4):
    """Ring state after a prefill of n tokens (``oracle/decode_engine.py:90-95``).

    kv_proj/score_proj: [n, 2d] fp32 projections of the prefill tokens.  Returns (kvs, scs),
    each [2*ratio, 2d]: slots 0..r-1 hold the last full group (score biased by ape), slots r..
    hold the remainder tokens (biased), the rest is kv=0 / score=-inf.
    """
    n, two_d = kv_proj.shape
    cut = n - n % ratio
    kvs = torch.zeros(2 * ratio, two_d)
    scs = torch.full((2 * ratio, two_d), float("-inf"))
    if cut >= ratio:
        kvs[:ratio] = kv_proj[cut - ratio:cut]
        scs[:ratio] = score_proj[cut - ratio:cut] + ape
    rem = n - cut
    if rem:
        kvs[ratio:ratio + rem] = kv_proj[cut:]
        scs[ratio:ratio + rem] = score_proj[cut:] + ape[:rem]
    return kvs, scs


def ring_step(kvs, scs, kv_p, score_p, pos, ape, norm_w, freqs, ratio=4, rope_head_dim=64,
              fp8_sim=True, eps=1e-6):
    """One decode token at position ``pos``.  kvs/scs: ring [2r, 2d] (updated in place);
    kv_p/score_p: [2d] projections of the token; freqs: [rd/2] fp32 angular frequencies of the
    compressed-row RoPE.  Returns the emitted compressed row [d] when (pos+1) % r == 0, else None.
    """
    slot = ratio + pos % ratio
    kvs[slot] = kv_p
    scs[slot] = score_p + ape[pos % ratio]
    if (pos + 1) % ratio != 0:
        return None
    two_d = kvs.shape[1]
    d = two_d // 2
    kv8 = torch.cat([kvs[:ratio, :d], kvs[ratio:, d:]], dim=0)          # [2r, d]
    sc8 = torch.cat([scs[:ratio, :d], scs[ratio:, d:]], dim=0)
    row = (kv8 * torch.softmax(sc8, dim=0)).sum(dim=0)
    row = norm_w * (row * torch.rsqrt(row.pow(2).mean() + eps))
    rd = rope_head_dim
    ang = (pos + 1 - ratio) * freqs
    cis = torch.polar(torch.ones_like(ang), ang)[None]
    rot = apply_rotary_emb(row[d - rd:][None, None], cis)[0, 0]
    row = torch.cat([row[: d - rd], rot])
    if fp8_sim:
        nope, _ = _fp8.act_quant_sim(row[: d - rd].numpy()[None], 64)
        row = torch.cat([torch.from_numpy(nope[0]), row[d - rd:]])
    kvs[:ratio] = kvs[ratio:].clone()
    scs[:ratio] = scs[ratio:].clone()
    return row


def mean_pool(kv, ratio=4):
    """kv:[b, n, d] -> [b, n//ratio, d]: fp32 sum of each block's rows in order, times 1/ratio."""
    b, n, d = kv.shape
    g = n // ratio
    blk = kv[:, : g * ratio].float().reshape(b, g, ratio, d)
    acc = blk[:, :, 0]
    for j in range(1, ratio):
        acc = acc + blk[:, :, j]
    return acc * (1.0 / ratio)
