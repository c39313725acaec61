"""RMSNorm, YaRN RoPE frequencies and interleaved-pair rotary embedding (CPU oracle).

Restates ``ref_torch/norm_rope.py``:

* ``rmsnorm``               — ``ref_torch/norm_rope.py:10-16``
* ``precompute_freqs``      — ``ref_torch/norm_rope.py:19-43``
* ``precompute_freqs_cis``  — ``ref_torch/norm_rope.py:46-50``
* ``apply_rotary_emb``      — ``ref_torch/norm_rope.py:53-62``
* ``rope_cos_sin``          — ``v4mlx/norm_rope.py:38-43`` (real cos/sin tables)

Pinning: golden vectors produced by ``tests/golden/make_golden.py`` from the reference
(``precompute_freqs_cis`` fp32 rounding, ``apply_rotary_emb``), the YaRN correction range closed
form (low/high = 15/25 for dim 64, base 1.6e5, original length 65536, beta 32/1), rotation
invariants (norm preservation per pair, inverse = conjugate) and the no-YaRN special case
``freqs = base**(-2i/dim)``.
"""
import math

import torch


def rmsnorm(x, weight, eps=1e-6):
    """Row RMS normalisation in fp32, scaled by ``weight``; result cast back to x's dtype."""
    xf = x.float()
    inv = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (weight * (xf * inv)).to(x.dtype)


def yarn_correction_range(dim, base, original_seq_len, beta_fast, beta_slow):
    """Integer [low, high] band of rotary dims that YaRN ramps between (clamped to [0, dim-1])."""
    def corr(rotations):
        return dim * math.log(original_seq_len / (rotations * 2 * math.pi)) / (2 * math.log(base))
    lo = math.floor(corr(beta_fast))
    hi = math.ceil(corr(beta_slow))
    return max(lo, 0), min(hi, dim - 1)


def precompute_freqs(dim, seqlen, original_seq_len, base, factor, beta_fast, beta_slow):
    """Per-pair angular frequency [dim/2] (fp32), YaRN-blended when original_seq_len > 0.

    ``seqlen`` is accepted for signature parity with the reference and does not affect the
    frequencies.
    """
    del seqlen
    exps = torch.arange(0, dim, 2, dtype=torch.float32) / dim
    freqs = 1.0 / (base ** exps)
    if original_seq_len > 0:
        lo, hi = yarn_correction_range(dim, base, original_seq_len, beta_fast, beta_slow)
        if lo == hi:
            hi = hi + 0.001
        ramp = ((torch.arange(dim // 2, dtype=torch.float32) - lo) / (hi - lo)).clamp(0, 1)
        keep = 1 - ramp                       # weight of the un-interpolated frequency
        freqs = freqs / factor * (1 - keep) + freqs * keep
    return freqs


def precompute_freqs_cis(dim, seqlen, original_seq_len, base, factor, beta_fast, beta_slow):
    """Unit complex rotations [seqlen, dim/2] (complex64) at integer positions 0..seqlen-1."""
    freqs = precompute_freqs(dim, seqlen, original_seq_len, base, factor, beta_fast, beta_slow)
    ang = torch.outer(torch.arange(seqlen), freqs)
    return torch.polar(torch.ones_like(ang), ang)


def rope_cos_sin(dim, seqlen, original_seq_len, base, factor, beta_fast, beta_slow):
    """Real (cos, sin) tables [seqlen, dim/2] of the same rotations, fp32."""
    cis = precompute_freqs_cis(dim, seqlen, original_seq_len, base, factor, beta_fast, beta_slow)
    return cis.real.contiguous(), cis.imag.contiguous()


def apply_rotary_emb(x, freqs_cis, inverse=False):
    """Rotate interleaved pairs (x0,x1),(x2,x3),... of the last dim by ``freqs_cis``.

    x: [b, s, dim] or [b, s, heads, dim]; freqs_cis: [s, dim/2] complex.  The rotation is the
    complex product (x0 + i x1) * e^{i theta} (conjugate when ``inverse``).
    """
    xf = x.float()
    pairs = xf.reshape(*xf.shape[:-1], -1, 2)
    re, im = pairs[..., 0], pairs[..., 1]
    c, s = freqs_cis.real, freqs_cis.imag
    if inverse:
        s = -s
    if xf.dim() == 3:
        c = c.reshape(1, c.shape[0], c.shape[-1])
        s = s.reshape(1, s.shape[0], s.shape[-1])
    else:
        c = c.reshape(1, c.shape[0], 1, c.shape[-1])
        s = s.reshape(1, s.shape[0], 1, s.shape[-1])
    out = torch.stack([re * c - im * s, re * s + im * c], dim=-1)
    return out.reshape(xf.shape).to(x.dtype)
