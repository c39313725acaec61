"""Drop-in sparse attention with the call signatures of ``ref_torch/sparse_attn.py``.

* ``get_window_topk_idxs(window_size, bsz, seqlen, start_pos)`` — ``ref_torch/sparse_attn.py:9-20``
  (built on the device; int32 instead of int64, same values and shapes: [bsz, 1, w] for decode,
  [bsz, seqlen, min(seqlen, w)] for prefill).
* ``sparse_attn(q, kv, attn_sink, topk_idxs, scale)`` — ``ref_torch/sparse_attn.py:23-34``,
  with an optional ``dv`` (value width; the 576-wide latent rows carry 512 value columns).
* ``sparse_attn_batched`` / ``sparse_attn_two_source`` — the same op over a batch of caches and
  over the engine's virtual [window; compressed] buffer (``oracle/decode_engine.py:108-115``)
  without building the concatenation.
* ``prefill_attn`` — the prompt's per-position loop (``oracle/decode_engine.py:107-117``) with the
  row sets computed on the device; ``decode_attn`` — the decode index build over indexer scores
  and the attention over it (``oracle/decode_engine.py:110-117``) in one call.

Everything runs in libsmla's HIP kernels; tensors must live on the GPU.
"""
import torch

from . import ops


def get_window_topk_idxs(window_size, bsz, seqlen, start_pos, device="cuda"):
    return ops.window_topk_idxs(window_size, bsz, seqlen, start_pos, device=device)


def sparse_attn(q, kv, attn_sink, topk_idxs, scale, dv=None):
    """q:[s,h,d], kv:[n,d], attn_sink:[h] (or None), topk_idxs:[s,T] (int, -1 = masked)
    -> o:[s,h,dv] (dv defaults to d) in q's dtype.  Out-of-range ids are masked."""
    if q.dim() != 3 or kv.dim() != 2 or topk_idxs.dim() != 2:
        raise ValueError("expected q [s,h,d], kv [n,d], topk_idxs [s,T]")
    if kv.shape[1] != q.shape[2] or topk_idxs.shape[0] != q.shape[0]:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, kv {tuple(kv.shape)}, idx {tuple(topk_idxs.shape)}")
    dv = q.shape[2] if dv is None else dv
    kv = kv.to(q.dtype) if kv.dtype not in (q.dtype, torch.uint8) and not _is_fp8(kv) else kv
    out = ops.sparse_attn_op(q[None], kv[None], None, None, None, attn_sink, topk_idxs[None], float(scale), dv)
    return out[0]


def _is_fp8(t):
    return hasattr(torch, "float8_e4m3fn") and t.dtype == torch.float8_e4m3fn


def sparse_attn_batched(q, kv, attn_sink, topk_idxs, scale, dv=None, kv_scale=None):
    """q:[B,s,h,d], kv:[B,n,d] (bf16/fp32, or fp8 codes with kv_scale [B,n,d/64]),
    topk_idxs:[B,s,T] -> [B,s,h,dv]."""
    dv = q.shape[-1] if dv is None else dv
    return ops.sparse_attn_op(q, kv, None, kv_scale, None, attn_sink, topk_idxs, float(scale), dv)


def prefill_attn(q, kv_raw, kv_comp, attn_sink, scale, q_pos0=0, window=128, ratio=4, dv=512, out_dtype=None):
    """Prompt attention of ``oracle/decode_engine.py:107-117`` without index lists: query s (position
    q_pos0 + s) attends raw rows max(0, p-window+1)..p and, for ratio > 0, the compressed rows
    0..(p+1)//ratio - 1 -- the same result, bit for bit, as ``sparse_attn_two_source`` over
    ``workloads.prefill_indices`` lists.  q [B,S,H,D] bf16, kv_raw [B,n_raw,D], kv_comp [B,n_comp,D]
    or None -> [B,S,H,dv] (q's dtype unless out_dtype is given)."""
    return ops.prefill_attn_op(q, kv_raw, kv_comp if ratio > 0 else None, attn_sink, int(q_pos0), int(window),
                               int(ratio), float(scale), int(dv), out_dtype or q.dtype)


def sparse_attn_two_source(q, kv0, kv1, attn_sink, topk_idxs, scale, dv=None, kv0_scale=None, kv1_scale=None):
    """Ids index the virtual concatenation [kv0; kv1] along rows (per batch entry)."""
    dv = q.shape[-1] if dv is None else dv
    return ops.sparse_attn_op(q, kv0, kv1, kv0_scale, kv1_scale, attn_sink, topk_idxs, float(scale), dv)


def decode_attn(q, kv_raw, kv_comp, attn_sink, scores, pos, window, k, scale, dv=512, nvis=None, out=None,
                workspace=None):
    """Decode attention over the index list ``select_decode_indices(scores, k, pos, window, n_raw,
    nvis)`` builds, without the list going through memory when the shape allows (the attention
    workgroups select the rows themselves) -- the same output, bit for bit, as that list followed by
    ``sparse_attn_two_source``.  q [B,1,H,D] (or [B,S,H,D] with scores/pos of B*S rows), kv_raw
    [B,n_raw,D], kv_comp [B,n_comp,D], scores [B*S,N] fp32, pos [B*S] int32 -> [B,S,H,dv]."""
    B, S, H, D = q.shape
    if out is None:
        out = torch.empty(B, S, H, dv, dtype=q.dtype if q.dtype in (torch.bfloat16, torch.float32) else torch.float32,
                          device=q.device)
    if workspace is None:
        workspace = torch.empty(ops.decode_attn_workspace(B, S, H, D, dv, window, k, q.dtype, kv_raw.dtype,
                                                          out.dtype), dtype=torch.uint8, device=q.device)
    return ops.decode_attn_into(q, kv_raw, kv_comp, attn_sink, scores, nvis, pos, window, k, scale, dv, out,
                                workspace)
