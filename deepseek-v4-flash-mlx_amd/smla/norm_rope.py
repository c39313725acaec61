"""RMSNorm and YaRN RoPE tables with the signatures of ``ref_torch/norm_rope.py``.

The rotation tables are host-side constants, computed once on the CPU in fp32 exactly as the
reference does (``torch.polar`` of ``outer(positions, freqs)``, ``ref_torch/norm_rope.py:46-50``)
and uploaded; the HIP kernels (compressor pooling, ring step) consume them as cos/sin arrays.
``rmsnorm``/``apply_rotary_emb`` are plain torch on the GPU for callers around the hot path.
"""
import functools
import math

import torch


def rmsnorm(x, weight, eps=1e-6):
    """``ref_torch/norm_rope.py:10-16``."""
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
    """``ref_torch/norm_rope.py:53-62``: rotate interleaved pairs by complex freqs."""
    xc = torch.view_as_complex(x.float().unflatten(-1, (-1, 2)))
    fc = freqs_cis.conj() if inverse else freqs_cis
    if xc.ndim == 3:
        fc = fc.view(1, xc.size(1), xc.size(-1))
    else:
        fc = fc.view(1, xc.size(1), 1, xc.size(-1))
    return torch.view_as_real(xc * fc).flatten(-2).to(x.dtype)
