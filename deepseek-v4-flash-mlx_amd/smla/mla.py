"""MLA projections with the signatures of ``v4mlx/mla.py``, on the GPU.

These dense GEMMs surround the sparse-attention core, with the reference's shapes: H=64 heads,
head_dim 512, rope 64, 8 output groups of rank 1024.  Every product runs in libsmla's HIP kernels
(``smla_linear`` / ``smla_o_proj``): up to 32 bf16 token rows (decode) the weight-streaming MFMA
kernel, bound by reading the weights once; larger batches (prefill) the tiled MFMA GEMM, with the
inverse RoPE of ``o_project`` fused into its operand load.  Every function refuses tensors that are
not on the GPU.
"""
import torch

from . import ops

N_HEADS, HEAD_DIM, ROPE_HD = 64, 512, 64
N_GROUPS, O_LORA = 8, 1024


def linear(x, W):
    """``v4mlx/mla.py:16-18``: y = x @ W^T, W [out, in] (bf16 or fp32 operands, the result in x's
    type)."""
    ops._on_gpu(x, W)
    if x.dtype != W.dtype or x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"linear: x ({x.dtype}) and W ({W.dtype}) must both be bf16 or both fp32")
    lead = x.shape[:-1]
    return ops.linear_op(x.reshape(-1, x.shape[-1]), W, 1, x.dtype).reshape(*lead, W.shape[0])


def q_down(x, wq_a):
    """``v4mlx/mla.py:21-23``."""
    return linear(x, wq_a)


def perhead_norm(q, eps=1e-6):
    """``v4mlx/mla.py:26-28``: weightless per-head RMS."""
    ops._on_gpu(q)
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
    ops._on_gpu(o, wo_a, wo_b)
    lead = o.shape[:-1]
    o3 = o.reshape(-1, N_GROUPS, o.shape[-1] // N_GROUPS)          # heads of a group as one slice
    y = ops.o_proj_op(o3, None, None, None, wo_a, wo_b, N_GROUPS, torch.bfloat16)
    return y.reshape(*lead, wo_b.shape[0])


def o_project(o, pos, cos_t, sin_t, wo_a, wo_b):
    """``oracle/decode_engine.py:118-119`` (up to the hc_post call): o [T, N_HEADS, HEAD_DIM] has the
    last ROPE_HD dims of every head rotated back to position 0 (inverse RoPE at pos [T], cos/sin
    tables [n_pos, ROPE_HD/2]), then goes through ``o_grouped``.  One HIP call (``smla_o_proj``),
    the rotation fused into the first product's operand load."""
    ops._on_gpu(o, pos, cos_t, sin_t, wo_a, wo_b)
    return ops.o_proj_op(o, pos, cos_t, sin_t, wo_a, wo_b, N_GROUPS, torch.bfloat16)
