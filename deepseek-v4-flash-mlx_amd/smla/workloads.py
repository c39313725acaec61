"""Seeded synthetic inputs for the sparse-MLA workloads (all drawn on the CPU with
``torch.Generator().manual_seed(seed)``, then cast: bf16 by round-to-nearest-even, fp8 by pow2
block scales + e4m3fn rounding).  Draw order within a workload is fixed: q, kv, q_idx, k_idx, w.

Workloads (names describe the shapes):
* ``fp32_plumbing``  — one decode step, fp32: H=16, rows [4096, 576], top-k 512 by an fp32
                       indexer (q_idx [16,64], keys [4096,64], weights 1), no sink, scale 1/24.
* ``decode_32k``     — B=8, H=64, raw latent [8, 32768, 576] bf16, block-4 mean pool to
                       [8, 8192, 576], fp8 indexer keys [8, 8192, 64] + per-row pow2 scale,
                       q_idx [8, 64, 64] bf16, weights [8, 64], top-k 2048 + 128-row window at
                       position 32767.
* ``prefill_4k``     — S=4096 queries, H=64, raw [4096, 576] + mean-pooled [1024, 576] bf16;
                       query p attends window max(0,p-127)..p and compressed rows [0, (p+1)//4).
* ``decode_64k``     — B=1, raw [65536, 576], compressed [16384, 576], fp8 keys [16384, 64],
                       20 steps from position 65516 (one raw row per step, a compressed row and
                       key every 4th).
* ``batched_fp8``    — B=64, lengths U{2048..16384}, e4m3 rows with per-64 pow2 scales,
                       2048 random sorted ids per sequence (all rows when fewer), H=64.
"""
import math

import torch

LATENT, ROPE, D, DV = 512, 64, 576, 512
SCALE_576 = 1.0 / math.sqrt(576.0)


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def pow2_scale(amax):
    """Exact 2**ceil(log2(amax / 448)) of fp32 amax (> 0)."""
    v = (amax / 448.0).float()
    m, e = torch.frexp(v)
    e = e - (m == 0.5).to(e.dtype)
    return torch.ldexp(torch.ones_like(v), e)


def quant_e4m3_pow2(x, block=64):
    """fp32 [..., n] -> (uint8 codes [..., n], fp32 scales [..., n/block])."""
    sh = x.shape
    blk = x.float().reshape(*sh[:-1], sh[-1] // block, block)
    amax = blk.abs().amax(-1).clamp_min(1e-4)
    s = pow2_scale(amax)
    z = (blk / s[..., None]).clamp(-448.0, 448.0)
    codes = z.to(torch.float8_e4m3fn).view(torch.uint8).reshape(sh)
    return codes, s


def dequant_e4m3(codes, scales, block=64):
    sh = codes.shape
    v = codes.view(torch.float8_e4m3fn).float().reshape(*sh[:-1], sh[-1] // block, block)
    return (v * scales[..., None]).reshape(sh)


def fp32_plumbing():
    g = _gen(0)
    q = torch.randn(1, 16, D, generator=g) * 0.1
    kv = torch.randn(4096, D, generator=g) * 0.1
    q_idx = torch.randn(1, 16, 64, generator=g)
    k_idx = torch.randn(4096, 64, generator=g)
    w = torch.ones(1, 16)
    return dict(q=q, kv=kv, q_idx=q_idx, k_idx=k_idx, w=w, k=512, scale=SCALE_576, dv=DV, sink=None)


def decode_32k(B=8, n_raw=32768, ratio=4, H=64, Hi=64, Di=64, k=2048, window=128, seed=1):
    g = _gen(seed)
    q = (torch.randn(B, 1, H, D, generator=g) * 0.05).to(torch.bfloat16)
    raw = (torch.randn(B, n_raw, D, generator=g) * 0.05).to(torch.bfloat16)
    q_idx = torch.randn(B, 1, Hi, Di, generator=g).to(torch.bfloat16)
    k_idx = torch.randn(B, n_raw // ratio, Di, generator=g)
    w = torch.randn(B, 1, Hi, generator=g)
    codes, kscale = quant_e4m3_pow2(k_idx, block=Di)
    return dict(q=q, raw=raw, q_idx=q_idx, k_codes=codes, kscale=kscale.reshape(B, -1), w=w, k=k,
                window=window, ratio=ratio, pos=n_raw - 1, scale=SCALE_576, dv=DV, sink=None)


def prefill_4k(S=4096, H=64, ratio=4, window=128, seed=2):
    g = _gen(seed)
    q = (torch.randn(1, S, H, D, generator=g) * 0.05).to(torch.bfloat16)
    raw = (torch.randn(1, S, D, generator=g) * 0.05).to(torch.bfloat16)
    return dict(q=q, raw=raw, ratio=ratio, window=window, scale=SCALE_576, dv=DV, sink=None)


def prefill_indices(S, ratio=4, window=128, n_raw=None, q_pos0=0):
    """[S, window + S//ratio] int32: ids into [raw; compressed] for queries at positions
    q_pos0..q_pos0+S-1 (window rows, then the causally visible compressed rows), -1 padded."""
    n_raw = S if n_raw is None else n_raw
    nc = (q_pos0 + S) // ratio
    T = window + nc
    p = torch.arange(q_pos0, q_pos0 + S).unsqueeze(1)
    j = torch.arange(window).unsqueeze(0)
    lo = (p - window + 1).clamp(min=0)
    wid = lo + j
    wid = torch.where(wid > p, torch.full_like(wid, -1), wid)
    c = torch.arange(nc).unsqueeze(0)
    cid = torch.where(c < (p + 1) // ratio, n_raw + c, torch.full_like(c, -1))
    return torch.cat([wid, cid], dim=1).to(torch.int32)[:, :T]


def decode_64k(n_raw=65536, ratio=4, H=64, Hi=64, Di=64, k=2048, window=128, steps=20, seed=3):
    g = _gen(seed)
    q = (torch.randn(steps, 1, H, D, generator=g) * 0.05).to(torch.bfloat16)
    raw = (torch.randn(1, n_raw, D, generator=g) * 0.05).to(torch.bfloat16)
    q_idx = torch.randn(steps, Hi, Di, generator=g).to(torch.bfloat16)
    k_idx = torch.randn(1, n_raw // ratio, Di, generator=g)
    w = torch.randn(steps, Hi, generator=g)
    codes, kscale = quant_e4m3_pow2(k_idx, block=Di)
    return dict(q=q, raw=raw, q_idx=q_idx, k_codes=codes, kscale=kscale.reshape(1, -1), w=w, k=k,
                window=window, ratio=ratio, pos0=n_raw - steps, steps=steps, scale=SCALE_576, dv=DV,
                sink=None)


def batched_fp8(B=64, lo=2048, hi=16384, H=64, k=2048, seed=4):
    g = _gen(seed)
    lens = torch.randint(lo, hi + 1, (B,), generator=g)
    q = (torch.randn(B, 1, H, D, generator=g) * 0.05).to(torch.bfloat16)
    nmax = int(lens.max())
    codes = torch.zeros(B, nmax, D, dtype=torch.uint8)
    scales = torch.ones(B, nmax, D // 64)
    for b in range(B):
        L = int(lens[b])
        x = torch.randn(L, D, generator=g) * 0.05
        c, s = quant_e4m3_pow2(x)
        codes[b, :L] = c
        scales[b, :L] = s
    idx = torch.full((B, 1, k), -1, dtype=torch.int32)
    for b in range(B):
        L = int(lens[b])
        sel = torch.randperm(L, generator=g)[:k].sort().values
        idx[b, 0, : sel.numel()] = sel.to(torch.int32)
    return dict(q=q, codes=codes, scales=scales, lens=lens, idx=idx, k=k, scale=SCALE_576, dv=DV, sink=None)
