"""KV compressor with the signatures of ``ref_torch/compressor.py``.

* ``overlap_transform(tensor, ratio, d, value)`` — ``ref_torch/compressor.py:12-18`` (a layout op,
  done with torch indexing on the device).
* ``compressor_prefill(x, wkv, wgate, ape, norm_w, ...)`` — ``ref_torch/compressor.py:21-50``:
  the two projections in one tiled MFMA GEMM over [wkv; wgate] (fp32 operands for fp32 inputs,
  bf16 for bf16), pooling + RMSNorm + RoPE in the HIP ``gated_pool`` kernel; returns (kv, state)
  like the reference.  ``fp8_sim`` adds the fp8 round trip of the
  non-rope channels (``v4mlx/compressor.py:60-62``); ``rotate`` the indexer compressor's
  Hadamard + fp4 round trip of all channels (``v4mlx/compressor.py:57-59``), in the same kernel.
* ``block_mean_pool(kv, ratio)`` — plain block mean, HIP.
* ``Ring`` — the decode-time compressor ring of ``oracle/decode_engine.py:90-105`` kept on the
  device: ``Ring.step`` writes the token, emits a row every ``ratio`` tokens straight into the
  caller's compressed cache (no host round trip), and shifts.
"""
import torch

from . import _lib, ops
from .norm_rope import rope_tables


def _sim(fp8_sim, rotate):
    return _lib.SIM_ROTATE_FP4 if rotate else _lib.SIM_FP8 if fp8_sim else _lib.SIM_NONE


def overlap_transform(tensor, ratio, d, value):
    ops._on_gpu(tensor)
    b, s = tensor.shape[0], tensor.shape[1]
    new = tensor.new_full((b, s, 2 * ratio, d), value)
    new[:, :, ratio:] = tensor[:, :, :, d:]
    new[:, 1:, :ratio] = tensor[:, :-1, :, :d]
    return new


def compressor_prefill(x, wkv, wgate, ape, norm_w, head_dim=512, ratio=4, rope_head_dim=64, base=160000.0,
                       original_seq_len=65536, factor=16, beta_fast=32, beta_slow=1, fp8_sim=False,
                       rotate=False):
    """x:[b,s,dim] -> (kv:[b, s//ratio, head_dim] fp32 post-RoPE, state dict)."""
    ops._on_gpu(x, wkv, wgate, ape, norm_w)
    b, s, _ = x.shape
    kv, score = project_pair(x, wkv, wgate)
    rem = s % ratio
    cut = s - rem
    state = {}
    if cut >= ratio:
        state["kv"] = kv[:, cut - ratio:cut].clone()
        state["score"] = (score[:, cut - ratio:cut] + ape.float()).clone()
    if rem > 0:
        state["kv_rem"] = kv[:, cut:].clone()
    if cut == 0:
        return kv.new_empty(b, 0, head_dim), state
    cos_t, sin_t = rope_tables(rope_head_dim, s, original_seq_len, base, factor, beta_fast, beta_slow,
                               device=x.device)
    out = ops.gated_pool_op(kv[:, :cut], score[:, :cut], ape, norm_w, cos_t, sin_t, ratio, rope_head_dim,
                            1e-6, _sim(fp8_sim, rotate))
    return out, state


def project_pair(x, wkv, wgate):
    """(x @ wkv^T, x @ wgate^T) as fp32 [b, s, 2*head_dim] each, from one ``smla_linear`` call over
    the stacked weights: fp32 operands unless x and both weights are bf16."""
    b, s, dim = x.shape
    wcat = torch.cat([wkv, wgate], dim=0)
    if x.dtype == torch.bfloat16 and wcat.dtype == torch.bfloat16:
        y = ops.linear_op(x.reshape(b * s, dim), wcat, 1, torch.float32)
    else:
        y = ops.linear_op(x.float().reshape(b * s, dim), wcat.float(), 1, torch.float32)
    y = y.reshape(b, s, -1)
    n = wkv.shape[0]
    return y[..., :n], y[..., n:]


def block_mean_pool(kv, ratio=4):
    """kv:[B,N,D] -> [B,N//ratio,D] (same dtype)."""
    return ops.block_mean_pool_op(kv, ratio)


class Ring:
    """Device-resident compressor ring for B sequences (``oracle/decode_engine.py:68-69,90-105``).

    ring_kv / ring_sc: [B, 2*ratio, 2*head_dim] fp32;  the compressed cache [B, cap, head_dim] fp32
    is owned by the caller and filled in place.
    """

    def __init__(self, B, head_dim, ape, norm_w, ratio=4, rope_head_dim=64, max_pos=65536, fp8_sim=True,
                 device="cuda", rope_args=(65536, 160000.0, 16, 32, 1), rotate=False):
        self.ratio, self.rd, self.sim = ratio, rope_head_dim, _sim(fp8_sim, rotate)
        self.ring_kv = torch.zeros(B, 2 * ratio, 2 * head_dim, device=device)
        self.ring_sc = torch.full((B, 2 * ratio, 2 * head_dim), float("-inf"), device=device)
        self.ape = ape.float().contiguous().to(device)
        self.norm_w = norm_w.float().contiguous().to(device)
        orig, base, factor, bf, bs = rope_args
        self.cos_t, self.sin_t = rope_tables(rope_head_dim, max_pos, orig, base, factor, bf, bs, device=device)

    def init_from_prefill(self, kv_proj, score_proj):
        """kv_proj/score_proj: [B, n, 2d] projections of the prefill tokens
        (``oracle/decode_engine.py:90-95``)."""
        B, n, _ = kv_proj.shape
        r = self.ratio
        cut = n - n % r
        self.ring_kv.zero_()
        self.ring_sc.fill_(float("-inf"))
        if cut >= r:
            self.ring_kv[:, :r] = kv_proj[:, cut - r:cut]
            self.ring_sc[:, :r] = score_proj[:, cut - r:cut] + self.ape
        rem = n - cut
        if rem:
            self.ring_kv[:, r:r + rem] = kv_proj[:, cut:]
            self.ring_sc[:, r:r + rem] = score_proj[:, cut:] + self.ape[:rem]

    def step(self, kv_p, score_p, pos, comp_cache):
        """kv_p/score_p: [B, 2d] projections of the token at positions pos [B] (int32, device)."""
        ops.ring_step_op(self.ring_kv, self.ring_sc, kv_p, score_p, pos, self.ape, self.norm_w, self.cos_t,
                         self.sin_t, self.ratio, self.rd, 1e-6, self.sim, comp_cache)
