"""MLA projections with the signatures of ``v4mlx/mla.py`` (torch on the GPU).

These dense GEMMs surround the sparse-attention core; they run as torch.matmul (hipBLASLt) with
the reference's shapes: H=64 heads, head_dim 512, rope 64, 8 output groups of rank 1024.
"""
import torch

N_HEADS, HEAD_DIM, ROPE_HD = 64, 512, 64
N_GROUPS, O_LORA = 8, 1024


def linear(x, W):
    """``v4mlx/mla.py:16-18``: y = x @ W^T, W [out, in]."""
    return x @ W.t()


def q_down(x, wq_a):
    """``v4mlx/mla.py:21-23``."""
    return linear(x, wq_a)


def perhead_norm(q, eps=1e-6):
    """``v4mlx/mla.py:26-28``: weightless per-head RMS."""
    return q * torch.rsqrt(q.square().mean(-1, keepdim=True) + eps)


def q_up(qln, wq_b):
    """``v4mlx/mla.py:31-34``: -> [..., N_HEADS, HEAD_DIM]."""
    q = linear(qln, wq_b)
    return q.reshape(*q.shape[:-1], N_HEADS, HEAD_DIM)


def kv_proj(x, wkv):
    """``v4mlx/mla.py:37-39``."""
    return linear(x, wkv)


def o_grouped(o, wo_a, wo_b):
    """``v4mlx/mla.py:42-56``: grouped low-rank output projection.
    o [..., N_HEADS*HEAD_DIM] -> [..., dim];  wo_a [N_GROUPS*O_LORA, N_HEADS*HEAD_DIM/N_GROUPS]."""
    lead = o.shape[:-1]
    og = o.reshape(-1, N_GROUPS, o.shape[-1] // N_GROUPS).transpose(0, 1).contiguous()   # [G, M, 4096]
    wa = wo_a.reshape(N_GROUPS, O_LORA, -1).transpose(1, 2).contiguous()                 # [G, 4096, 1024]
    ob = torch.bmm(og, wa)                                                              # [G, M, 1024]
    ob = ob.transpose(0, 1).reshape(*lead, N_GROUPS * O_LORA)
    return linear(ob, wo_b)
