"""MLA projections with the signatures of ``v4mlx/mla.py``, on the GPU.

These dense GEMMs surround the sparse-attention core, with the reference's shapes: H=64 heads,
head_dim 512, rope 64, 8 output groups of rank 1024.  Decode shapes (at most 32 token rows, bf16)
run the HIP projection kernel (``smla_linear`` / ``smla_o_proj``: MFMA, bound by streaming the
weights once); larger batches (prefill) run torch.matmul (hipBLASLt).  Every function refuses
tensors that are not on the GPU.
"""
import torch

from . import ops

_MAX_DECODE_ROWS = 32


def _decode_shape(x, *ws, k_mult=512):
    rows = x.numel() // x.shape[-1] if x.dim() else 0
    return (x.is_cuda and 0 < rows <= _MAX_DECODE_ROWS and x.dtype == torch.bfloat16
            and all(w.dtype == torch.bfloat16 for w in ws) and x.shape[-1] % k_mult == 0)

N_HEADS, HEAD_DIM, ROPE_HD = 64, 512, 64
N_GROUPS, O_LORA = 8, 1024


def linear(x, W):
    """``v4mlx/mla.py:16-18``: y = x @ W^T, W [out, in]."""
    ops._on_gpu(x, W)
    if _decode_shape(x, W) and W.shape[0] % 16 == 0:
        lead = x.shape[:-1]
        return ops.linear_op(x.reshape(-1, x.shape[-1]), W, 1, torch.bfloat16).reshape(*lead, W.shape[0])
    return x @ W.t()


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
    if _decode_shape(o, wo_a, wo_b, k_mult=512 * N_GROUPS):
        o3 = o.reshape(-1, N_GROUPS, o.shape[-1] // N_GROUPS)          # heads of a group as one slice
        y = ops.o_proj_op(o3, None, None, None, wo_a, wo_b, N_GROUPS, torch.bfloat16)
        return y.reshape(*lead, wo_b.shape[0])
    og = o.reshape(-1, N_GROUPS, o.shape[-1] // N_GROUPS).transpose(0, 1).contiguous()   # [G, M, 4096]
    wa = wo_a.reshape(N_GROUPS, O_LORA, -1).transpose(1, 2).contiguous()                 # [G, 4096, 1024]
    ob = torch.bmm(og, wa)                                                              # [G, M, 1024]
    ob = ob.transpose(0, 1).reshape(*lead, N_GROUPS * O_LORA)
    return linear(ob, wo_b)


def o_project(o, pos, cos_t, sin_t, wo_a, wo_b):
    """``oracle/decode_engine.py:118-119`` (up to the hc_post call): o [T, N_HEADS, HEAD_DIM] has the
    last ROPE_HD dims of every head rotated back to position 0 (inverse RoPE at pos [T], cos/sin
    tables [n_pos, ROPE_HD/2]), then goes through ``o_grouped``.  One fused HIP path for decode
    shapes; an in-place HIP rotation of a copy plus the GEMMs otherwise."""
    ops._on_gpu(o, pos, cos_t, sin_t, wo_a, wo_b)
    T = o.shape[0]
    if _decode_shape(o.reshape(T, -1), wo_a, wo_b, k_mult=512 * N_GROUPS):
        return ops.o_proj_op(o, pos, cos_t, sin_t, wo_a, wo_b, N_GROUPS, torch.bfloat16)
    r = o.contiguous().clone()
    ops.rope_op_(r, pos, cos_t, sin_t, True)
    return o_grouped(r.reshape(T, -1), wo_a, wo_b)
