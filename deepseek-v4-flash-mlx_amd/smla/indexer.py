"""Indexer scoring and top-k selection over compressed positions (HIP).

The reference has no indexer: its engine attends every causally visible compressed row
(``oracle/decode_engine.py:112-114``).  ``indexer_score`` implements the build's definition
(ReLU-gated per-head dot products, per-head weights, per-key scale, one fixed fp32 order) and
``topk`` the exact selection (score desc, index asc, ascending output, -1 padding), which equals
the reference's index build whenever the visible count is at most k.
"""
import torch

from . import ops


def indexer_score(q_idx, keys, kscale, weights, nvis=None):
    """q_idx [B,S,Hi,Di], keys [B,N,Di] (fp32/bf16/fp8 codes), kscale [B,N] or None,
    weights [B,S,Hi], nvis [B,S] or None -> [B,S,N] fp32."""
    return ops.indexer_score_op(q_idx, keys, kscale, weights, nvis)


def indexer_score_fp4(q_idx, codes, block_scales, kscale, weights, nvis=None):
    """The same scores over keys stored as packed e2m1 codes [B,N,Di/2] and ue8m0 scales
    [B,N,Di/32] (the form ``qat.fp4_quantize`` and ``smla_rotate_fp4`` write), bit-identical to
    ``indexer_score`` on the decoded fp32 keys."""
    return ops.indexer_score_fp4_op(q_idx, codes, block_scales, kscale, weights, nvis)


def topk(scores, k, nvis=None, id_offset=0):
    """scores [..., N] -> int32 [..., k]."""
    return ops.topk_op(scores, k, nvis, id_offset)


def select_decode_indices(scores, k, pos, window, n_raw, out=None, nvis=None):
    """The decode attention index list per sequence: the raw-cache window rows pos-window+1..pos
    (columns 0..window-1) followed by the top-k compressed rows offset by ``n_raw`` (the raw
    cache length, so ids index the virtual [raw; compressed] buffer), ranked among the first
    nvis[b] scores of each row (all N when nvis is None).
    scores [B, N] fp32, pos [B] int32, nvis [B] int32 or None -> out [B, window + k] int32."""
    B = scores.shape[0]
    if out is None:
        out = torch.empty(B, window + k, dtype=torch.int32, device=scores.device)
    ops.select_decode_into(scores.contiguous(), k, pos, window, out, id_offset=n_raw, nvis=nvis)
    return out


def index_decode(q_idx, keys, kscale, weights, nvis, k, pos, window, n_raw, out=None, workspace=None, flags=0):
    """Indexer scores and the decode index list in one call: ``indexer_score`` into the workspace
    followed by ``select_decode_indices`` (the same list, bit for bit).
    q_idx [B,1,Hi,Di], keys [B,N,Di], kscale [B,N] or None, weights [B,1,Hi], nvis [B,1] or None,
    pos [B] int32 -> out [B, window + k] int32.  flags: 0 or ``_lib.INDEX_EXACT`` (the same
    output: the scores are always the fixed-order ones)."""
    B, S = q_idx.shape[:2]
    N = keys.shape[1]
    if out is None:
        out = torch.empty(B * S, window + k, dtype=torch.int32, device=q_idx.device)
    if workspace is None:
        workspace = torch.empty(ops.index_decode_workspace(B, S, N), dtype=torch.uint8, device=q_idx.device)
    ops.index_decode_into(q_idx, keys, kscale, weights, nvis, k, pos if window > 0 else None, window, out,
                          workspace, id_offset=n_raw, flags=flags)
    return out
