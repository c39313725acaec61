"""RMSNorm and YaRN RoPE tables with the signatures of ``ref_torch/norm_rope.py``.

The rotation tables are host-side constants, computed once on the CPU in fp32 exactly as the
reference does (``torch.polar`` of ``outer(positions, freqs)``, ``ref_torch/norm_rope.py:46-50``)
and uploaded; the HIP kernels (compressor pooling, ring step, ``smla_rope``) consume them as cos/sin
arrays.  ``apply_rotary_emb`` runs ``smla_rope``; ``rmsnorm`` is plain torch on the GPU for callers
around the hot path.  Both refuse tensors that are not on the GPU.
"""
import functools
import math

import torch

from . import ops


def rmsnorm(x, weight, eps=1e-6):
    """``ref_torch/norm_rope.py:10-16``."""
    ops._on_gpu(x, weight)
    xf = x.float()
    return (weight * (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps))).to(x.dtype)


def precompute_freqs(dim, seqlen, original_seq_len, base, factor, beta_fast, beta_slow):
    """``ref_torch/norm_rope.py:19-43``: per-pair frequencies [dim/2], YaRN-ramped."""
    freqs = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    if original_seq_len > 0:
        def corr(rot):
            return dim * math.log(original_seq_len / (rot * 2 * math.pi)) / (2 * math.log(base))
        lo = max(math.floor(corr(beta_fast)), 0)
        hi = min(math.ceil(corr(beta_slow)), dim - 1)
        if lo == hi:
            hi += 0.001
        ramp = torch.clamp((torch.arange(dim // 2, dtype=torch.float32) - lo) / (hi - lo), 0, 1)
        smooth = 1 - ramp
        freqs = freqs / factor * (1 - smooth) + freqs * smooth
    return freqs


def precompute_freqs_cis(dim, seqlen, original_seq_len, base, factor, beta_fast, beta_slow):
    """``ref_torch/norm_rope.py:46-50``: complex64 [seqlen, dim/2]."""
    freqs = precompute_freqs(dim, seqlen, original_seq_len, base, factor, beta_fast, beta_slow)
    ang = torch.outer(torch.arange(seqlen), freqs)
    return torch.polar(torch.ones_like(ang), ang)


@functools.lru_cache(maxsize=16)
def _tables_cpu(dim, seqlen, original_seq_len, base, factor, beta_fast, beta_slow):
    cis = precompute_freqs_cis(dim, seqlen, original_seq_len, base, factor, beta_fast, beta_slow)
    return cis.real.contiguous(), cis.imag.contiguous()


_DEVICE_TABLES = {}


def rope_tables(dim, seqlen, original_seq_len=65536, base=160000.0, factor=16, beta_fast=32, beta_slow=1,
                device="cuda"):
    """(cos, sin) fp32 [seqlen, dim/2] on ``device`` (cached)."""
    key = (dim, seqlen, original_seq_len, float(base), factor, beta_fast, beta_slow, str(device))
    if key not in _DEVICE_TABLES:
        c, s = _tables_cpu(dim, seqlen, original_seq_len, float(base), factor, beta_fast, beta_slow)
        _DEVICE_TABLES[key] = (c.to(device), s.to(device))
    return _DEVICE_TABLES[key]


def apply_rotary_emb(x, freqs_cis, inverse=False):
    """``ref_torch/norm_rope.py:53-62``: rotate the interleaved pairs of x [b, s, dim] or
    [b, s, heads, dim] by freqs_cis [s, dim/2] (row i for sequence position i), conjugated when
    ``inverse``; returns a new tensor of x's dtype.  Runs ``smla_rope`` (each product and sum
    rounded in float32, then rounded to x's dtype) on a copy of x."""
    ops._on_gpu(x, freqs_cis)
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("apply_rotary_emb takes fp32 or bf16")
    b, s = x.shape[0], x.shape[1]
    d = x.shape[-1]
    heads = x.shape[2] if x.dim() == 4 else 1
    y = x.contiguous().clone().reshape(b * s, heads, d)
    cos_t, sin_t = freqs_cis.real.float().contiguous(), freqs_cis.imag.float().contiguous()
    pos = torch.arange(s, dtype=torch.int32, device=x.device).repeat(b)
    ops.rope_op_(y, pos, cos_t, sin_t, bool(inverse))
    return y.reshape(x.shape)
