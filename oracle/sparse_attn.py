"""Window indices and dense-gather sparse attention with an attention sink (CPU oracle).

Restates:

* ``get_window_topk_idxs`` — ``ref_torch/sparse_attn.py:9-20`` (ring branch, partial branch,
  prefill causal band);
* ``sparse_attn``          — ``ref_torch/sparse_attn.py:23-34``: gather ``kv[idx]`` (idx < 0 is
  masked), ``scores = scale * q . kv``, softmax over the valid rows with ``exp(sink - rowmax)``
  added to the denominator, output = weighted sum of the gathered rows.  Duplicate indices count
  twice; a query with no valid index yields NaN (``-inf - -inf``), as in the reference;
* ``engine_decode_idxs``   — the engine's per-position index build, window ∪ causally visible
  compressed rows of the concatenated [window; compressed] buffer
  (``oracle/decode_engine.py:110-114``).

With 576-wide rows (512 latent + 64 rope) and a 512-wide value, each output column depends only
on the same column of the gathered rows, so the value output is ``sparse_attn(...)[..., :512]``;
``dv`` selects that slice.

Pinning: closed forms (T=1 gives ``kv_row * e^x / (e^x + e^sink)``), equality with
``torch.nn.functional.scaled_dot_product_attention`` on per-query gathered rows when the sink is
``-inf`` (a library routine), invariance under permutation of the index list, ``-1`` ≡ removal,
duplicate counting, a brute-force per-(query, head) loop on tiny shapes, and brute-force
enumeration of every window-index branch.
"""
import torch


def get_window_topk_idxs(window_size, bsz, seqlen, start_pos):
    """Window index matrix of the reference, expanded over the batch.

    * decode with a full ring (start_pos >= window-1): the ring slots in age order,
      [p+1, ..., w-1, 0, ..., p] with p = start_pos % w;  shape [bsz, 1, w].
    * decode with a partial window (0 < start_pos < w-1): [0..start_pos] then -1 padding;
      shape [bsz, 1, w].
    * prefill (start_pos == 0): row i holds max(0, i-w+1) + j for j < min(seqlen, w), with -1
      where that exceeds i;  shape [bsz, seqlen, min(seqlen, w)].

    (The reference expands a 1-D decode row with ``expand(bsz, -1, -1)``, which prepends the
    batch dimension to [1, w].)
    """
    w = window_size
    if start_pos >= w - 1:
        p = start_pos % w
        ring = [(p + 1 + j) % w for j in range(w)]
        mat = torch.tensor(ring, dtype=torch.int64)
    elif start_pos > 0:
        mat = torch.full((w,), -1, dtype=torch.int64)
        mat[: start_pos + 1] = torch.arange(start_pos + 1)
    else:
        cols = min(seqlen, w)
        i = torch.arange(seqlen).unsqueeze(1)
        lo = (i - w + 1).clamp(min=0)
        mat = lo + torch.arange(cols).unsqueeze(0)
        mat = torch.where(mat > i, torch.full_like(mat, -1), mat)
    if mat.dim() == 1:
        mat = mat.unsqueeze(0)
    return mat.unsqueeze(0).expand(bsz, *mat.shape)


def engine_decode_idxs(pos, n_window_rows, n_comp, ratio, window=128):
    """Index list of the engine for query position ``pos`` over the buffer
    [window rows (n_window_rows, oldest first); compressed rows (n_comp)].

    Window part: positions max(0, pos-window+1)..pos mapped to their row in the window buffer
    (row = position - max(0, pos-window+1) when the buffer holds exactly those rows, which is how
    the engine lays it out).  Compressed part: the first min(n_comp, (pos+1)//ratio) compressed
    rows, offset by n_window_rows.  ratio 0 means no compressed rows.
    """
    lo = max(0, pos - window + 1)
    widx = list(range(pos + 1 - lo))
    nvis = (pos + 1) // ratio if ratio else 0
    cidx = [n_window_rows + j for j in range(min(n_comp, nvis))]
    return torch.tensor(widx + cidx, dtype=torch.int32)


def sparse_attn(q, kv, attn_sink, topk_idxs, scale, dv=None, chunk=64):
    """q:[s,h,d], kv:[n,d], attn_sink:[h] (or None = -inf), topk_idxs:[s,T] -> o:[s,h,dv].

    Computed in fp32 on upcast inputs, ``chunk`` queries at a time to bound the gathered
    [chunk, T, d] buffer.
    """
    q = q.float()
    kv = kv.float()
    s, h, d = q.shape
    dv = d if dv is None else dv
    sink = (torch.full((h,), float("-inf")) if attn_sink is None else attn_sink.float())
    idx_all = topk_idxs.long()
    out = torch.empty(s, h, dv, dtype=torch.float32)
    for c0 in range(0, s, chunk):
        c1 = min(s, c0 + chunk)
        idx = idx_all[c0:c1]
        valid = idx >= 0
        rows = kv[idx.clamp(min=0)]                                   # [c, T, d]
        logits = torch.bmm(q[c0:c1], rows.transpose(1, 2).contiguous()) * scale   # [c, h, T]
        logits = logits.masked_fill(~valid[:, None, :], float("-inf"))
        m = logits.amax(dim=-1, keepdim=True)                         # [c, h, 1]
        p = torch.exp(logits - m)
        den = p.sum(dim=-1, keepdim=True) + torch.exp(sink.view(1, h, 1) - m)
        out[c0:c1] = torch.bmm(p, rows[..., :dv].contiguous()) / den
    return out


def sparse_attn_batched(q, kv, attn_sink, topk_idxs, scale, dv=None):
    """Batched form: q:[B,s,h,d], kv:[B,n,d], topk_idxs:[B,s,T] -> [B,s,h,dv]."""
    return torch.stack([sparse_attn(q[b], kv[b], attn_sink, topk_idxs[b], scale, dv)
                        for b in range(q.shape[0])])


def sparse_attn_bruteforce(q, kv, attn_sink, topk_idxs, scale, dv=None):
    """Per-(query, head) loop over the index list in float64 — tiny shapes only."""
    q = q.double()
    kv = kv.double()
    s, h, d = q.shape
    dv = d if dv is None else dv
    out = torch.empty(s, h, dv, dtype=torch.float64)
    for i in range(s):
        ids = [int(t) for t in topk_idxs[i] if int(t) >= 0]
        for hh in range(h):
            if not ids:
                out[i, hh] = float("nan")
                continue
            lg = [float(scale * (q[i, hh] @ kv[t])) for t in ids]
            m = max(lg)
            ws = [torch.exp(torch.tensor(x - m, dtype=torch.float64)) for x in lg]
            sink = float("-inf") if attn_sink is None else float(attn_sink[hh])
            den = sum(ws) + torch.exp(torch.tensor(sink - m, dtype=torch.float64))
            acc = torch.zeros(dv, dtype=torch.float64)
            for wgt, t in zip(ws, ids):
                acc += wgt * kv[t, :dv]
            out[i, hh] = acc / den
    return out
