"""torch.library custom ops over libsmla (GPU only; no CPU fallback inside any op).

Each op validates shapes/dtypes on the host, allocates its outputs (and workspace) with torch's
caching allocator, and launches on ``torch.cuda.current_stream()``.  Fake (meta) kernels give
output shapes for tracing.
"""
from typing import Optional

import torch

from . import _lib

_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16,
       torch.uint8: _lib.FP8_E4M3}
if hasattr(torch, "float8_e4m3fn"):
    _DT[torch.float8_e4m3fn] = _lib.FP8_E4M3


def dtype_code(t):
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def _p(t):
    return None if t is None else t.data_ptr()


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _on_gpu(*ts):
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("smla ops run on the GPU only (got a tensor on %s)" % t.device)


def _c(t):
    return None if t is None else t.contiguous()


# ----------------------------------------------------------------------------------------------
def _is_fp8_rows(t):
    return t.dtype == torch.uint8 or (hasattr(torch, "float8_e4m3fn") and t.dtype == torch.float8_e4m3fn)


_YDT_ATTN = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}


def _check_attn(q, kv0, kv1, kv0_scale, kv1_scale, attn_sink, topk_idxs, dv):
    """Shape and type agreement of the attention operands, checked before any launch (a mismatch
    would send the kernel's row, index or scale addressing past its buffers)."""
    if q.dim() != 4 or kv0.dim() != 3 or topk_idxs.dim() != 3:
        raise ValueError("expected q [B,S,H,D], kv0 [B,n0,D], topk_idxs [B,S,T]")
    B, S, H, D = q.shape
    if kv0.shape[0] != B or kv0.shape[2] != D:
        raise ValueError(f"kv0 {tuple(kv0.shape)} does not match q {tuple(q.shape)}: expected [{B}, n0, {D}]")
    if kv1 is not None:
        if kv1.dim() != 3 or kv1.shape[0] != B or kv1.shape[2] != D:
            raise ValueError(f"kv1 {tuple(kv1.shape)} does not match q {tuple(q.shape)}: expected [{B}, n1, {D}]")
        if kv1.dtype != kv0.dtype:
            raise ValueError(f"kv1 dtype {kv1.dtype} differs from kv0's {kv0.dtype}")
    if topk_idxs.shape[0] != B or topk_idxs.shape[1] != S:
        raise ValueError(f"topk_idxs {tuple(topk_idxs.shape)} does not match q: expected [{B}, {S}, T]")
    if not 0 < dv <= D:
        raise ValueError(f"dv={dv} must lie in 1..{D}")
    if attn_sink is not None and tuple(attn_sink.shape) != (H,):
        raise ValueError(f"attn_sink {tuple(attn_sink.shape)} must be [{H}]")
    if _is_fp8_rows(kv0):
        if D % 64 != 0:
            raise ValueError("fp8 rows need D % 64 == 0")
        for kv, sc, name in ((kv0, kv0_scale, "kv0_scale"), (kv1, kv1_scale, "kv1_scale")):
            if kv is None:
                continue
            if sc is None or tuple(sc.shape) != (B, kv.shape[1], D // 64) or sc.dtype != torch.float32:
                got = None if sc is None else (tuple(sc.shape), sc.dtype)
                raise ValueError(f"{name} must be fp32 [{B}, {kv.shape[1]}, {D // 64}], got {got}")
    elif kv0_scale is not None or kv1_scale is not None:
        raise ValueError("scales are given for fp8 rows only")


def _attn_args(q, kv0, kv1, kv0_scale, kv1_scale, attn_sink, topk_idxs, dv):
    _on_gpu(q, kv0, kv1, kv0_scale, kv1_scale, attn_sink, topk_idxs)
    _check_attn(q, kv0, kv1, kv0_scale, kv1_scale, attn_sink, topk_idxs, dv)
    q, kv0, kv1 = q.contiguous(), kv0.contiguous(), _c(kv1)
    kv0_scale, kv1_scale, attn_sink = _c(kv0_scale), _c(kv1_scale), _c(attn_sink)
    if topk_idxs.dtype != torch.int32:
        topk_idxs = topk_idxs.to(torch.int32)
    topk_idxs = topk_idxs.contiguous()
    if attn_sink is not None and attn_sink.dtype != torch.float32:
        attn_sink = attn_sink.float()
    return q, kv0, kv1, kv0_scale, kv1_scale, attn_sink, topk_idxs


def attn_plan(B, S, H, D, dv, T, q_dtype=torch.bfloat16, kv_dtype=torch.bfloat16, out_dtype=None,
              rows_per_split=0):
    """(nsplit, rows_per_split, workspace bytes) of the attention path's split plan for these sizes
    (``smla_sparse_attn_plan``); rows_per_split 0 asks for the default plan."""
    import ctypes
    ns, rps = ctypes.c_int64(0), ctypes.c_int64(0)
    qd, kd = _DT[q_dtype], _DT[kv_dtype]
    od = _DT[out_dtype if out_dtype is not None else q_dtype]
    wsb = _lib.lib().smla_sparse_attn_plan(B, S, H, D, dv, T, qd, kd, od, rows_per_split, ctypes.byref(ns),
                                           ctypes.byref(rps))
    return ns.value, rps.value, int(wsb)


@torch.library.custom_op("smla::prefill_attn", mutates_args=(), device_types="cuda")
def prefill_attn_op(q: torch.Tensor, kv_raw: torch.Tensor, kv_comp: Optional[torch.Tensor],
                    attn_sink: Optional[torch.Tensor], q_pos0: int, window: int, ratio: int, scale: float,
                    dv: int, out_dtype: torch.dtype) -> torch.Tensor:
    """q [B,S,H,D] bf16 at positions q_pos0..q_pos0+S-1, kv_raw [B,n_raw,D] bf16, kv_comp
    [B,n_comp,D] bf16 or None -> [B,S,H,dv]: every query attends its window rows and the compressed
    rows causally visible to it (the row sets are computed in the kernel)."""
    _on_gpu(q, kv_raw, kv_comp, attn_sink)
    if q.dim() != 4 or kv_raw.dim() != 3:
        raise ValueError("expected q [B,S,H,D] and kv_raw [B,n_raw,D]")
    B, S, H, D = q.shape
    if kv_raw.shape[0] != B or kv_raw.shape[2] != D:
        raise ValueError(f"kv_raw {tuple(kv_raw.shape)} does not match q {tuple(q.shape)}")
    if kv_comp is not None and (kv_comp.dim() != 3 or kv_comp.shape[0] != B or kv_comp.shape[2] != D):
        raise ValueError(f"kv_comp {tuple(kv_comp.shape)} does not match q {tuple(q.shape)}")
    if attn_sink is not None and tuple(attn_sink.shape) != (H,):
        raise ValueError(f"attn_sink {tuple(attn_sink.shape)} must be [{H}]")
    if q.dtype != torch.bfloat16 or kv_raw.dtype != torch.bfloat16 or (kv_comp is not None and
                                                                      kv_comp.dtype != torch.bfloat16):
        raise TypeError("prefill_attn takes bf16 q and rows")
    q, kv_raw, kv_comp = q.contiguous(), kv_raw.contiguous(), _c(kv_comp)
    if attn_sink is not None:
        attn_sink = attn_sink.float().contiguous()
    n_comp = kv_comp.shape[1] if kv_comp is not None else 0
    out = torch.empty(B, S, H, dv, dtype=out_dtype, device=q.device)
    _lib.call("smla_prefill_attn", _p(q), _lib.BF16, _p(kv_raw), kv_raw.shape[1], _p(kv_comp), n_comp, _lib.BF16,
              _p(attn_sink), int(q_pos0), int(window), int(ratio), B, S, H, D, dv, float(scale), _p(out),
              _YDT_ATTN[out_dtype], _stream(q))
    return out


@prefill_attn_op.register_fake
def _(q, kv_raw, kv_comp, attn_sink, q_pos0, window, ratio, scale, dv, out_dtype):
    return q.new_empty(*q.shape[:3], dv, dtype=out_dtype)


@torch.library.custom_op("smla::sparse_attn", mutates_args=(), device_types="cuda")
def sparse_attn_op(q: torch.Tensor, kv0: torch.Tensor, kv1: Optional[torch.Tensor],
                   kv0_scale: Optional[torch.Tensor], kv1_scale: Optional[torch.Tensor],
                   attn_sink: Optional[torch.Tensor], topk_idxs: torch.Tensor, scale: float,
                   dv: int) -> torch.Tensor:
    """q [B,S,H,D], kv0 [B,n0,D], kv1 [B,n1,D]|None, scales [B,n,D/64] (fp8 rows),
    attn_sink [H]|None, topk_idxs [B,S,T] -> out [B,S,H,dv] in q's dtype."""
    q, kv0, kv1, kv0_scale, kv1_scale, attn_sink, topk_idxs = _attn_args(q, kv0, kv1, kv0_scale, kv1_scale,
                                                                         attn_sink, topk_idxs, dv)
    B, S, H, D = q.shape
    T = topk_idxs.shape[-1]
    n0 = kv0.shape[1]
    n1 = 0 if kv1 is None else kv1.shape[1]
    out = torch.empty(B, S, H, dv, dtype=q.dtype, device=q.device)
    qd, kd, od = dtype_code(q), dtype_code(kv0), dtype_code(out)
    wsb = _lib.lib().smla_sparse_attn_workspace(B, S, H, D, dv, T, qd, kd)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=q.device)
    _lib.call("smla_sparse_attn", _p(q), qd, _p(kv0), n0, _p(kv1), n1, kd, _p(kv0_scale),
              _p(kv1_scale), _p(attn_sink), _p(topk_idxs), T, B, S, H, D, dv, float(scale),
              _p(out), od, _p(ws), wsb, _stream(q))
    return out


def sparse_attn_ex(q, kv0, kv1, kv0_scale, kv1_scale, attn_sink, topk_idxs, scale, dv, rows_per_split=0,
                   phases=3, out=None, workspace=None):
    """``smla_sparse_attn_ex``: the attention op with an explicit split plan (rows_per_split, 0 =
    default) and a choice of launches (phases: 1 split kernel, 2 merge, 3 both), into `out` and
    `workspace` when given (no allocation then).  Returns out."""
    q, kv0, kv1, kv0_scale, kv1_scale, attn_sink, topk_idxs = _attn_args(q, kv0, kv1, kv0_scale, kv1_scale,
                                                                         attn_sink, topk_idxs, dv)
    B, S, H, D = q.shape
    T = topk_idxs.shape[-1]
    n0 = kv0.shape[1]
    n1 = 0 if kv1 is None else kv1.shape[1]
    if out is None:
        out = torch.empty(B, S, H, dv, dtype=q.dtype, device=q.device)
    elif tuple(out.shape) != (B, S, H, dv) or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous [{B}, {S}, {H}, {dv}] tensor")
    _on_gpu(out)
    qd, kd, od = dtype_code(q), dtype_code(kv0), dtype_code(out)
    _, _, wsb = attn_plan(B, S, H, D, dv, T, q.dtype, kv0.dtype, out.dtype, rows_per_split)
    if workspace is None:
        workspace = torch.empty(max(wsb, 1), dtype=torch.uint8, device=q.device)
    _on_gpu(workspace)
    have = workspace.numel() * workspace.element_size()
    _lib.call("smla_sparse_attn_ex", _p(q), qd, _p(kv0), n0, _p(kv1), n1, kd, _p(kv0_scale), _p(kv1_scale),
              _p(attn_sink), _p(topk_idxs), T, B, S, H, D, dv, float(scale), _p(out), od, int(rows_per_split),
              int(phases), _p(workspace), have, _stream(q))
    return out


@sparse_attn_op.register_fake
def _(q, kv0, kv1, kv0_scale, kv1_scale, attn_sink, topk_idxs, scale, dv):
    B, S, H, _D = q.shape
    return q.new_empty(B, S, H, dv)


# ----------------------------------------------------------------------------------------------
@torch.library.custom_op("smla::indexer_score", mutates_args=(), device_types="cuda")
def indexer_score_op(q: torch.Tensor, keys: torch.Tensor, kscale: Optional[torch.Tensor],
                     weights: torch.Tensor, nvis: Optional[torch.Tensor]) -> torch.Tensor:
    """q [B,S,Hi,Di] f32|bf16, keys [B,N,Di] f32|bf16|fp8, kscale [B,N]|None, weights [B,S,Hi],
    nvis [B,S]|None -> scores [B,S,N] fp32 (-inf past nvis)."""
    _on_gpu(q, keys, kscale, weights, nvis)
    q, keys, kscale, weights = q.contiguous(), keys.contiguous(), _c(kscale), weights.float().contiguous()
    if nvis is not None:
        nvis = nvis.to(torch.int32).contiguous()
    if kscale is not None:
        kscale = kscale.float().contiguous()
    B, S, Hi, Di = q.shape
    N = keys.shape[1]
    out = torch.empty(B, S, N, dtype=torch.float32, device=q.device)
    _lib.call("smla_indexer_score", _p(q), dtype_code(q), _p(keys), dtype_code(keys), _p(kscale),
              _p(weights), _p(nvis), B, S, Hi, Di, N, _p(out), _stream(q))
    return out


@indexer_score_op.register_fake
def _(q, keys, kscale, weights, nvis):
    return q.new_empty(q.shape[0], q.shape[1], keys.shape[1], dtype=torch.float32)


@torch.library.custom_op("smla::indexer_score_fp4", mutates_args=(), device_types="cuda")
def indexer_score_fp4_op(q: torch.Tensor, codes: torch.Tensor, block_scales: torch.Tensor,
                         kscale: Optional[torch.Tensor], weights: torch.Tensor,
                         nvis: Optional[torch.Tensor]) -> torch.Tensor:
    """q [B,S,Hi,Di] f32|bf16, codes [B,N,Di/2] uint8 (packed e2m1), block_scales [B,N,Di/32] uint8
    (ue8m0), kscale [B,N]|None, weights [B,S,Hi], nvis [B,S]|None -> scores [B,S,N] fp32."""
    _on_gpu(q, codes, block_scales, kscale, weights, nvis)
    B, S, Hi, Di = q.shape
    N = codes.shape[1]
    if codes.dtype != torch.uint8 or block_scales.dtype != torch.uint8:
        raise ValueError("fp4 keys are uint8 codes and uint8 ue8m0 block scales")
    if tuple(codes.shape) != (B, N, Di // 2) or tuple(block_scales.shape) != (B, N, Di // 32):
        raise ValueError(f"fp4 keys {tuple(codes.shape)} / scales {tuple(block_scales.shape)} do not match "
                         f"q {tuple(q.shape)}")
    q, codes, block_scales, weights = q.contiguous(), codes.contiguous(), block_scales.contiguous(), \
        weights.float().contiguous()
    if nvis is not None:
        nvis = nvis.to(torch.int32).contiguous()
    if kscale is not None:
        kscale = kscale.float().contiguous()
    out = torch.empty(B, S, N, dtype=torch.float32, device=q.device)
    _lib.call("smla_indexer_score_fp4", _p(q), dtype_code(q), _p(codes), _p(block_scales), _p(kscale),
              _p(weights), _p(nvis), B, S, Hi, Di, N, _p(out), _stream(q))
    return out


@indexer_score_fp4_op.register_fake
def _(q, codes, block_scales, kscale, weights, nvis):
    return q.new_empty(q.shape[0], q.shape[1], codes.shape[1], dtype=torch.float32)


# ----------------------------------------------------------------------------------------------
@torch.library.custom_op("smla::topk", mutates_args=(), device_types="cuda")
def topk_op(scores: torch.Tensor, k: int, nvis: Optional[torch.Tensor], id_offset: int) -> torch.Tensor:
    """scores [..., N] fp32 -> [..., k] int32 ascending ids (+ id_offset), -1 padded."""
    _on_gpu(scores, nvis)
    scores = scores.float().contiguous()
    N = scores.shape[-1]
    R = scores.numel() // N
    if nvis is not None:
        nvis = nvis.to(torch.int32).contiguous()
    out = torch.empty(*scores.shape[:-1], k, dtype=torch.int32, device=scores.device)
    _lib.call("smla_topk", _p(scores), R, N, _p(nvis), k, _p(out), k, int(id_offset), _stream(scores))
    return out


@topk_op.register_fake
def _(scores, k, nvis, id_offset):
    return scores.new_empty(*scores.shape[:-1], k, dtype=torch.int32)


# ----------------------------------------------------------------------------------------------
@torch.library.custom_op("smla::block_mean_pool", mutates_args=(), device_types="cuda")
def block_mean_pool_op(x: torch.Tensor, ratio: int) -> torch.Tensor:
    """x [B,N,D] -> [B,N//ratio,D] in x's dtype (fp32 sum in row order, times 1/ratio)."""
    _on_gpu(x)
    x = x.contiguous()
    B, N, D = x.shape
    out = torch.empty(B, N // ratio, D, dtype=x.dtype, device=x.device)
    _lib.call("smla_block_mean_pool", _p(x), dtype_code(x), B, N, D, ratio, _p(out), dtype_code(out),
              _stream(x))
    return out


@block_mean_pool_op.register_fake
def _(x, ratio):
    return x.new_empty(x.shape[0], x.shape[1] // ratio, x.shape[2])


# ----------------------------------------------------------------------------------------------
@torch.library.custom_op("smla::gated_pool", mutates_args=(), device_types="cuda")
def gated_pool_op(kv: torch.Tensor, score: torch.Tensor, ape: torch.Tensor, norm_w: torch.Tensor,
                  cos_t: torch.Tensor, sin_t: torch.Tensor, ratio: int, rope_head_dim: int, eps: float,
                  sim: int) -> torch.Tensor:
    """kv, score [B,N,2d] fp32 (N % ratio == 0) -> [B,N//ratio,d] fp32.  sim: 0 none, 1 fp8 of the
    non-rope channels, 2 Hadamard + fp4 of all channels (``_lib.SIM_*``)."""
    _on_gpu(kv, score, ape, norm_w, cos_t, sin_t)
    kv, score = kv.float().contiguous(), score.float().contiguous()
    ape, norm_w = ape.float().contiguous(), norm_w.float().contiguous()
    cos_t, sin_t = cos_t.float().contiguous(), sin_t.float().contiguous()
    B, N, two_d = kv.shape
    d = two_d // 2
    if cos_t.shape[0] < N:
        raise ValueError("rotation tables must cover every token position")
    out = torch.empty(B, N // ratio, d, dtype=torch.float32, device=kv.device)
    _lib.call("smla_gated_pool", _p(kv), _p(score), _p(ape), _p(norm_w), _p(cos_t), _p(sin_t), B, N, d,
              ratio, rope_head_dim, float(eps), int(sim), _p(out), _stream(kv))
    return out


@gated_pool_op.register_fake
def _(kv, score, ape, norm_w, cos_t, sin_t, ratio, rope_head_dim, eps, sim):
    return kv.new_empty(kv.shape[0], kv.shape[1] // ratio, kv.shape[2] // 2, dtype=torch.float32)


# ----------------------------------------------------------------------------------------------
@torch.library.custom_op("smla::ring_step", mutates_args=("ring_kv", "ring_sc", "comp_cache"),
                         device_types="cuda")
def ring_step_op(ring_kv: torch.Tensor, ring_sc: torch.Tensor, kv_p: torch.Tensor, score_p: torch.Tensor,
                 pos: torch.Tensor, ape: torch.Tensor, norm_w: torch.Tensor, cos_t: torch.Tensor,
                 sin_t: torch.Tensor, ratio: int, rope_head_dim: int, eps: float, sim: int,
                 comp_cache: torch.Tensor) -> None:
    """In-place decode ring update for B sequences; appends emitted rows to comp_cache [B,cap,d]."""
    _on_gpu(ring_kv, ring_sc, kv_p, score_p, pos, ape, norm_w, cos_t, sin_t, comp_cache)
    for t in (ring_kv, ring_sc, comp_cache):
        if not t.is_contiguous() or t.dtype != torch.float32:
            raise ValueError("ring and cache tensors must be contiguous fp32")
    B = ring_kv.shape[0]
    d = ring_kv.shape[-1] // 2
    # row-strided fp32 views (slices of one wider projection) pass as they are; anything else is packed
    # (8-byte aligned with an even row stride: the kernel moves two channels per access)
    strided = (kv_p.dtype == score_p.dtype == torch.float32 and kv_p.dim() == score_p.dim() == 2
               and kv_p.stride(1) == score_p.stride(1) == 1 and kv_p.stride(0) == score_p.stride(0)
               and kv_p.stride(0) % 2 == 0 and kv_p.data_ptr() % 8 == 0 and score_p.data_ptr() % 8 == 0)
    if not strided:
        kv_p, score_p = kv_p.float().contiguous(), score_p.float().contiguous()
    ld = kv_p.stride(0) if kv_p.dim() == 2 else 0
    pos = pos.to(torch.int32).contiguous()
    _lib.call("smla_ring_step", _p(ring_kv), _p(ring_sc), _p(kv_p), _p(score_p), _p(pos),
              _p(ape.float().contiguous()), _p(norm_w.float().contiguous()), _p(cos_t.float().contiguous()),
              _p(sin_t.float().contiguous()), cos_t.shape[0], B, d, ratio, rope_head_dim, float(eps),
              int(sim), _p(comp_cache), comp_cache.shape[1], ld, _stream(ring_kv))


@ring_step_op.register_fake
def _(ring_kv, ring_sc, kv_p, score_p, pos, ape, norm_w, cos_t, sin_t, ratio, rope_head_dim, eps, sim,
      comp_cache):
    return None


# ----------------------------------------------------------------------------------------------
@torch.library.custom_op("smla::quant_fp8_pow2", mutates_args=(), device_types="cuda")
def quant_fp8_pow2_op(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x [..., D] (D % 64 == 0) -> (codes uint8 [..., D], scales fp32 [..., D/64])."""
    _on_gpu(x)
    x = x.contiguous()
    D = x.shape[-1]
    rows = x.numel() // D
    codes = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    scales = torch.empty(*x.shape[:-1], D // 64, dtype=torch.float32, device=x.device)
    _lib.call("smla_quant_fp8_pow2", _p(x), dtype_code(x), rows, D, _p(codes), _p(scales), _stream(x))
    return codes, scales


@quant_fp8_pow2_op.register_fake
def _(x):
    return (x.new_empty(x.shape, dtype=torch.uint8),
            x.new_empty(*x.shape[:-1], x.shape[-1] // 64, dtype=torch.float32))


# ----------------------------------------------------------------------------------------------
@torch.library.custom_op("smla::rotate_fp4", mutates_args=(), device_types="cuda")
def rotate_fp4_op(x: torch.Tensor, rotate: bool, fp4: bool, want_out: bool,
                  want_codes: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """x [..., n] fp32/bf16 (n a power of two, 32..1024) -> (out fp32 [..., n], packed e2m1 codes
    uint8 [..., n/2], ue8m0 scales uint8 [..., n/32]); outputs not asked for come back empty."""
    _on_gpu(x)
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("rotate_fp4 takes fp32 or bf16")
    if want_codes and not fp4:
        raise ValueError("the stored form is the fp4 one")
    x = x.contiguous()
    n = x.shape[-1]
    rows = x.numel() // n if n else 0
    out = torch.empty(x.shape if want_out else (0,), dtype=torch.float32, device=x.device)
    codes = torch.empty((*x.shape[:-1], n // 2) if want_codes else (0,), dtype=torch.uint8, device=x.device)
    scales = torch.empty((*x.shape[:-1], n // 32) if want_codes else (0,), dtype=torch.uint8, device=x.device)
    flags = (_lib.QAT_ROTATE if rotate else 0) | (_lib.QAT_FP4 if fp4 else 0)
    _lib.call("smla_rotate_fp4", _p(x), dtype_code(x), rows, n, flags, _p(out) if want_out else None,
              _p(codes) if want_codes else None, _p(scales) if want_codes else None, _stream(x))
    return out, codes, scales


@rotate_fp4_op.register_fake
def _(x, rotate, fp4, want_out, want_codes):
    n = x.shape[-1]
    return (x.new_empty(x.shape if want_out else (0,), dtype=torch.float32),
            x.new_empty((*x.shape[:-1], n // 2) if want_codes else (0,), dtype=torch.uint8),
            x.new_empty((*x.shape[:-1], n // 32) if want_codes else (0,), dtype=torch.uint8))


# ----------------------------------------------------------------------------------------------
_YDT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}


@torch.library.custom_op("smla::linear", mutates_args=(), device_types="cuda")
def linear_op(x: torch.Tensor, w: torch.Tensor, groups: int, out_dtype: torch.dtype) -> torch.Tensor:
    """x [T, G*K], w [G*N, K] (both bf16 or both fp32) -> y [T, G*N]: y[:, gN:(g+1)N] = x[:, gK:(g+1)K] @ w_g^T
    (the weight-streaming kernel up to 32 bf16 rows, the tiled MFMA GEMM otherwise)."""
    _on_gpu(x, w)
    x, w = x.contiguous(), w.contiguous()
    T = x.shape[0]
    K = w.shape[1]
    N = w.shape[0] // groups
    if x.shape[1] != groups * K or w.shape[0] != groups * N:
        raise ValueError("linear: x [T, G*K] and w [G*N, K] do not agree")
    y = torch.empty(T, groups * N, dtype=out_dtype, device=x.device)
    _lib.call("smla_linear", _p(x), dtype_code(x), _p(w), dtype_code(w), T, groups, N, K, _p(y), _YDT[out_dtype],
              _stream(x))
    return y


@linear_op.register_fake
def _(x, w, groups, out_dtype):
    return x.new_empty(x.shape[0], w.shape[0], dtype=out_dtype)


@torch.library.custom_op("smla::rope_", mutates_args=("x",), device_types="cuda")
def rope_op_(x: torch.Tensor, pos: torch.Tensor, cos_t: torch.Tensor, sin_t: torch.Tensor, inverse: bool) -> None:
    """In place: the last rd = 2 * cos_t.shape[1] dims of every head of x [T, heads, head_dim]."""
    _on_gpu(x, pos, cos_t, sin_t)
    if not x.is_contiguous() or x.dim() != 3:
        raise ValueError("rope_: x must be a contiguous [T, heads, head_dim] tensor")
    pos = pos.to(torch.int32).contiguous()
    cos_t, sin_t = cos_t.float().contiguous(), sin_t.float().contiguous()
    T, H, D = x.shape
    _lib.call("smla_rope", _p(x), dtype_code(x), T, H, D, 2 * cos_t.shape[1], _p(pos), _p(cos_t), _p(sin_t),
              cos_t.shape[0], int(bool(inverse)), _stream(x))


@rope_op_.register_fake
def _(x, pos, cos_t, sin_t, inverse):
    return None


@torch.library.custom_op("smla::o_proj", mutates_args=(), device_types="cuda")
def o_proj_op(o: torch.Tensor, pos: Optional[torch.Tensor], cos_t: Optional[torch.Tensor],
              sin_t: Optional[torch.Tensor], wo_a: torch.Tensor, wo_b: torch.Tensor, groups: int,
              out_dtype: torch.dtype) -> torch.Tensor:
    """o [T, heads, head_dim] bf16 -> [T, dim]: inverse RoPE of the rope dims at pos (when given),
    grouped projection by wo_a [G*R, heads*head_dim/G], then wo_b [dim, G*R] (any T)."""
    tensors = [o, wo_a, wo_b] + ([pos, cos_t, sin_t] if pos is not None else [])
    _on_gpu(*tensors)
    o, wo_a, wo_b = o.contiguous(), wo_a.contiguous(), wo_b.contiguous()
    T, H, D = o.shape
    R = wo_a.shape[0] // groups
    dim = wo_b.shape[0]
    mid = torch.empty(T, groups * R, dtype=torch.bfloat16, device=o.device)
    y = torch.empty(T, dim, dtype=out_dtype, device=o.device)
    rd = n_pos = 0
    if pos is not None:
        pos = pos.to(torch.int32).contiguous()
        cos_t, sin_t = cos_t.float().contiguous(), sin_t.float().contiguous()
        rd, n_pos = 2 * cos_t.shape[1], cos_t.shape[0]
    _lib.call("smla_o_proj", _p(o), dtype_code(o), _p(pos), _p(cos_t), _p(sin_t), n_pos, T, H, D, rd, groups, R,
              _p(wo_a), _p(wo_b), dtype_code(wo_a), dim, _p(mid), _p(y), _YDT[out_dtype], _stream(o))
    return y


@o_proj_op.register_fake
def _(o, pos, cos_t, sin_t, wo_a, wo_b, groups, out_dtype):
    return o.new_empty(o.shape[0], wo_b.shape[0], dtype=out_dtype)


# ----------------------------------------------------------------------------------------------
def window_topk_idxs(window_size, bsz, seqlen, start_pos, device="cuda"):
    """Device-built window index matrix (int32); see sparse_attn.get_window_topk_idxs."""
    if start_pos > 0:
        out = torch.empty(bsz, 1, window_size, dtype=torch.int32, device=device)
    else:
        out = torch.empty(bsz, seqlen, min(seqlen, window_size), dtype=torch.int32, device=device)
    _on_gpu(out)
    _lib.call("smla_window_topk_idxs", window_size, bsz, seqlen, start_pos, _p(out), _stream(out))
    return out


def decode_window_idxs(pos, window, out=None):
    """pos [R] int32 (device) -> out [R, window] int32 with pos-window+1..pos (-1 where < 0)."""
    _on_gpu(pos)
    pos = pos.to(torch.int32).contiguous()
    R = pos.numel()
    stride = window
    if out is None:
        out = torch.empty(R, window, dtype=torch.int32, device=pos.device)
    else:
        stride = out.stride(0)
    _lib.call("smla_decode_window_idxs", _p(pos), R, window, _p(out), stride, _stream(pos))
    return out


def _check_row_epilogue(x, norm_w, pos, cos_t, rd, out, rows_per_pos, cache_rows):
    """Sizes the row epilogue's kernel relies on (the C entry cannot see tensor extents): one
    position per rows_per_pos input rows, a norm weight per channel, rd/2 table columns, and room
    in out for every row (row r, or row pos mod cache_rows of sequence r // rows_per_pos)."""
    rows, d = (x.shape[0], x.shape[-1]) if x.dim() == 2 else (x.numel() // x.shape[-1], x.shape[-1])
    if rows_per_pos < 1 or rows % rows_per_pos:
        raise ValueError(f"row_epilogue: {rows} rows are not a whole number of {rows_per_pos}-row positions")
    seqs = rows // rows_per_pos
    if pos is not None and pos.numel() != seqs:
        raise ValueError(f"row_epilogue: pos must hold {seqs} positions, got {pos.numel()}")
    if (rd or cache_rows) and pos is None:
        raise ValueError("row_epilogue: RoPE and the cache write need positions")
    if norm_w is not None and norm_w.numel() != d:
        raise ValueError(f"row_epilogue: norm_w must hold {d} weights, got {norm_w.numel()}")
    if rd and (cos_t is None or cos_t.dim() != 2 or cos_t.shape[1] != rd // 2):
        raise ValueError(f"row_epilogue: cos/sin tables must be [n_pos, {rd // 2}]")
    need = seqs * cache_rows * d if cache_rows > 0 else rows * d
    if out.numel() < need:
        raise ValueError(f"row_epilogue: out holds {out.numel()} elements, the rows need {need}")


def _check_decode_ids(B, ncomp, T, ids, comp32, comp_out):
    """The id list and the emitted-row copy address ids [B, T] and comp32 / comp_out [B, ncomp, d]."""
    if ids is not None and (ids.dtype != torch.int32 or not ids.is_contiguous() or tuple(ids.shape) != (B, T)):
        raise ValueError(f"ids must be a contiguous int32 [{B}, {T}] tensor")
    if (comp32 is None) != (comp_out is None):
        raise ValueError("comp32 and comp_out go together")
    if comp32 is not None:
        for t in (comp32, comp_out):
            if t.dim() != 3 or tuple(t.shape[:2]) != (B, ncomp) or not t.is_contiguous():
                raise ValueError(f"comp32 / comp_out must be contiguous [{B}, {ncomp}, d] tensors")
        if comp32.shape != comp_out.shape:
            raise ValueError("comp32 and comp_out must have the same shape")


def row_epilogue(x, norm_w, pos, cos_t, sin_t, rd, sim, out, rows_per_pos=1, cache_rows=0, eps=1e-6):
    """``smla_row_epilogue``: rows of x [rows, d] fp32 -> RMSNorm (norm_w [d], or None for the
    weightless norm) -> RoPE of the last rd channels at pos[row // rows_per_pos] -> `sim` -> out
    (bf16 or fp32): row r of out [rows, d], or with cache_rows > 0 row pos mod cache_rows of
    sequence r // rows_per_pos of a cache [.., cache_rows, d].  Stream-ordered; returns out."""
    _check_row_epilogue(x, norm_w, pos, cos_t, rd, out, rows_per_pos, cache_rows)
    _on_gpu(x, out, *(t for t in (norm_w, pos, cos_t, sin_t) if t is not None))
    if x.dtype != torch.float32 or x.stride(-1) != 1 or not out.is_contiguous():
        raise ValueError("row_epilogue: x must be fp32 with unit column stride and out contiguous")
    if x.dim() != 2:
        x = x.reshape(-1, x.shape[-1])
    d = x.shape[-1]
    rows = x.shape[0]
    ldx = x.stride(0)
    n_pos = cos_t.shape[0] if cos_t is not None else 0
    _lib.call("smla_row_epilogue", _p(x), rows, d, ldx, rows_per_pos, _p(pos), _p(norm_w), _p(cos_t), _p(sin_t),
              n_pos, rd, float(eps), int(sim), _p(out), dtype_code(out), cache_rows, _stream(x))
    return out


def row_epilogue_ids(x, norm_w, pos, cos_t, sin_t, rd, sim, out, rows_per_pos, ids_pos, window, ratio, n_raw,
                     ncomp, T, ids, comp32=None, comp_out=None, cache_rows=0, eps=1e-6):
    """``smla_row_epilogue_ids``: ``row_epilogue(x, norm_w, pos, cos_t, sin_t, rd, sim, out,
    rows_per_pos, cache_rows, eps)`` on rows of d = 512 and ``decode_ids(ids_pos, window, ratio,
    n_raw, ncomp, T, ids, comp32, comp_out)`` in one launch, bit for bit the two calls' results."""
    _check_row_epilogue(x, norm_w, pos, cos_t, rd, out, rows_per_pos, cache_rows)
    _check_decode_ids(ids_pos.numel(), ncomp, T, ids, comp32, comp_out)
    _on_gpu(x, out, ids_pos, ids, *(t for t in (norm_w, pos, cos_t, sin_t, comp32, comp_out) if t is not None))
    if x.dtype != torch.float32 or x.stride(-1) != 1 or not out.is_contiguous():
        raise ValueError("row_epilogue_ids: x must be fp32 with unit column stride and out contiguous")
    if x.dim() != 2:
        x = x.reshape(-1, x.shape[-1])
    ids_pos = ids_pos.to(torch.int32).contiguous()
    B = ids_pos.numel()
    n_pos = cos_t.shape[0] if cos_t is not None else 0
    d_comp = comp32.shape[-1] if comp32 is not None else 0
    _lib.call("smla_row_epilogue_ids", _p(x), x.shape[0], x.shape[-1], x.stride(0), rows_per_pos, _p(pos), _p(norm_w),
              _p(cos_t), _p(sin_t), n_pos, rd, float(eps), int(sim), _p(out), dtype_code(out), cache_rows,
              _p(ids_pos), B, window, ratio, n_raw, ncomp, _p(ids), T, _p(comp32), _p(comp_out), d_comp, _stream(x))
    return out, ids


def ring_step_kv(ring, kv_p, score_p, pos, comp_cache, kv_x, kv_norm, cos_t, sin_t, rd, sim, kv_cache,
                 cache_rows=None, eps=1e-6):
    """``smla_ring_step_kv``: ``ring.step(kv_p, score_p, pos, comp_cache)`` and
    ``row_epilogue(kv_x, kv_norm, pos, cos_t, sin_t, rd, sim, kv_cache, cache_rows=cache_rows)`` in
    one launch (``oracle/decode_engine.py:81-84,96-105``), bit for bit the two calls' results.
    kv_p/score_p [B, 2d] and kv_x [B, d] fp32: row-strided views pass as they are when 8-byte aligned
    with even row strides (slices of one projection), anything else is packed.  kv_cache
    [B, rows, d] bf16/fp32; cache_rows defaults to its rows.  Stream-ordered."""
    B0 = ring.ring_kv.shape[0]
    if pos.numel() != B0:
        raise ValueError(f"ring_step_kv: pos must hold {B0} positions, got {pos.numel()}")
    if cache_rows is not None and not 0 < cache_rows <= kv_cache.shape[1]:
        raise ValueError(f"ring_step_kv: cache_rows must lie in 1..{kv_cache.shape[1]}")
    _on_gpu(kv_p, score_p, pos, comp_cache, kv_x, kv_norm, cos_t, sin_t, kv_cache, ring.ring_kv)
    for t in (ring.ring_kv, ring.ring_sc, comp_cache):
        if not t.is_contiguous() or t.dtype != torch.float32:
            raise ValueError("ring and compressed-cache tensors must be contiguous fp32")
    if not kv_cache.is_contiguous():
        raise ValueError("kv_cache must be contiguous")
    B = ring.ring_kv.shape[0]
    d = ring.ring_kv.shape[-1] // 2
    if kv_cache.shape[0] != B or kv_cache.shape[-1] != d or comp_cache.shape[0] != B:
        raise ValueError(f"kv_cache and comp_cache must hold {B} sequences of {d}-wide rows")

    def rows(t, w):
        if (t.dtype != torch.float32 or t.dim() != 2 or tuple(t.shape) != (B, w) or t.stride(1) != 1
                or t.stride(0) % 2 or t.data_ptr() % 8):
            t = t.float().reshape(B, w).contiguous()
        return t

    kv_p, score_p, kv_x = rows(kv_p, 2 * d), rows(score_p, 2 * d), rows(kv_x, d)
    if kv_p.stride(0) != score_p.stride(0):
        kv_p, score_p = kv_p.contiguous(), score_p.contiguous()
    pos = pos.to(torch.int32).contiguous()
    kv_norm = kv_norm.float().contiguous()
    cos_t, sin_t = cos_t.float().contiguous(), sin_t.float().contiguous()
    _lib.call("smla_ring_step_kv", _p(ring.ring_kv), _p(ring.ring_sc), _p(kv_p), _p(score_p), _p(pos), _p(ring.ape),
              _p(ring.norm_w), _p(ring.cos_t), _p(ring.sin_t), ring.cos_t.shape[0], B, d, ring.ratio, ring.rd, 1e-6,
              int(ring.sim), _p(comp_cache), comp_cache.shape[1], kv_p.stride(0), _p(kv_x), kv_x.stride(0),
              _p(kv_norm), _p(cos_t), _p(sin_t), cos_t.shape[0], rd, float(eps), int(sim), _p(kv_cache),
              dtype_code(kv_cache), kv_cache.shape[1] if cache_rows is None else cache_rows, _stream(kv_p))


def decode_ids(pos, window, ratio, n_raw, ncomp, T, out=None, comp32=None, comp_out=None):
    """``smla_decode_ids``: [B, T] int32 ids (window rows, then the visible compressed rows offset
    by n_raw); with comp32/comp_out, an emitted compressed row is copied to bf16."""
    _check_decode_ids(pos.numel(), ncomp, T, out, comp32, comp_out)
    _on_gpu(pos, *(t for t in (out, comp32, comp_out) if t is not None))
    pos = pos.to(torch.int32).contiguous()
    B = pos.numel()
    if out is None:
        out = torch.empty(B, T, dtype=torch.int32, device=pos.device)
    d = comp32.shape[-1] if comp32 is not None else 0
    _lib.call("smla_decode_ids", _p(pos), B, window, ratio, n_raw, ncomp, _p(out), T, _p(comp32), _p(comp_out), d,
              _stream(pos))
    return out


def select_decode_into(scores, k, pos, window, out, id_offset=0, nvis=None):
    """Window ids then top-k ids per row, in one launch: scores [R, N], pos [R] int32,
    out int32 [R, >= window + k] (row stride out.stride(0))."""
    _on_gpu(scores, pos, out, nvis)
    if out.dtype != torch.int32 or out.stride(-1) != 1:
        raise ValueError("out must be an int32 view with unit inner stride")
    R, N = scores.shape
    if nvis is not None:
        nvis = nvis.to(torch.int32).contiguous()
    pos = pos.to(torch.int32).contiguous()
    _lib.call("smla_select_decode", _p(scores), R, N, _p(nvis), k, _p(pos), window, _p(out), out.stride(0),
              int(id_offset), _stream(scores))
    return out


def decode_attn_workspace(B, S, H, D, dv, window, k, q_dtype=torch.bfloat16, kv_dtype=torch.bfloat16,
                          out_dtype=torch.bfloat16):
    """Bytes of workspace smla_decode_attn needs."""
    return int(_lib.lib().smla_decode_attn_workspace(B, S, H, D, dv, window, k, _DT[q_dtype], _DT[kv_dtype],
                                                      _YDT_ATTN[out_dtype]))


def decode_attn_into(q, kv_raw, kv_comp, attn_sink, scores, nvis, pos, window, k, scale, dv, out, workspace):
    """The decode index build and the attention over it in one call (smla_decode_attn): q [B,S,H,D],
    kv_raw [B,n_raw,D], kv_comp [B,n_comp,D], attn_sink [H]|None, scores [B*S, N] fp32, nvis
    [B*S]|None, pos [B*S] int32, out [B,S,H,dv] (bf16 or fp32), workspace a uint8 tensor of at least
    decode_attn_workspace(...) bytes.  Same output as select_decode_into + sparse_attn_two_source."""
    _on_gpu(q, kv_raw, kv_comp, attn_sink, scores, nvis, pos, out, workspace)
    if q.dim() != 4 or kv_raw.dim() != 3 or kv_comp.dim() != 3 or scores.dim() != 2:
        raise ValueError("expected q [B,S,H,D], kv_raw / kv_comp [B,n,D], scores [B*S,N]")
    B, S, H, D = q.shape
    for name, kv in (("kv_raw", kv_raw), ("kv_comp", kv_comp)):
        if kv.shape[0] != B or kv.shape[2] != D:
            raise ValueError(f"{name} {tuple(kv.shape)} does not match q {tuple(q.shape)}")
    if kv_comp.dtype != kv_raw.dtype:
        raise TypeError("kv_raw and kv_comp must share a dtype")
    R, N = scores.shape
    if R != B * S or scores.dtype != torch.float32:
        raise ValueError(f"scores must be fp32 [{B * S}, N], got {tuple(scores.shape)} {scores.dtype}")
    if tuple(pos.shape) != (R,) or (nvis is not None and tuple(nvis.shape) != (R,)):
        raise ValueError("pos (and nvis) must be [B*S]")
    if attn_sink is not None and tuple(attn_sink.shape) != (H,):
        raise ValueError(f"attn_sink {tuple(attn_sink.shape)} must be [{H}]")
    if tuple(out.shape) != (B, S, H, dv) or out.dtype not in _YDT_ATTN or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous [{B},{S},{H},{dv}] bf16 or fp32 tensor")
    need = decode_attn_workspace(B, S, H, D, dv, window, k, q.dtype, kv_raw.dtype, out.dtype)
    if workspace.dtype != torch.uint8 or workspace.numel() < need:
        raise ValueError(f"workspace must be a uint8 tensor of at least {need} bytes")
    q, kv_raw, kv_comp, scores = q.contiguous(), kv_raw.contiguous(), kv_comp.contiguous(), scores.contiguous()
    if attn_sink is not None:
        attn_sink = attn_sink.float().contiguous()
    if nvis is not None:
        nvis = nvis.to(torch.int32).contiguous()
    pos = pos.to(torch.int32).contiguous()
    _lib.call("smla_decode_attn", _p(q), dtype_code(q), _p(kv_raw), kv_raw.shape[1], _p(kv_comp), kv_comp.shape[1],
              dtype_code(kv_raw), _p(attn_sink), _p(scores), N, _p(nvis), _p(pos), int(window), int(k), B, S, H, D,
              dv, float(scale), _p(out), _YDT_ATTN[out.dtype], _p(workspace), workspace.numel(), _stream(q))
    return out


def index_decode_workspace(B, S, N):
    """Bytes of workspace smla_index_decode needs for B*S query rows over N keys."""
    return int(_lib.lib().smla_index_decode_workspace(B, S, N))


def index_decode_into(q, keys, kscale, weights, nvis, k, pos, window, out, workspace, id_offset=0, flags=0):
    """Indexer scores and the decode index build in one call (smla_index_decode): q [B,S,Hi,Di],
    keys [B,N,Di], kscale [B,N]|None, weights [B,S,Hi], nvis [B,S]|None, pos [B*S] int32 (None
    when window == 0), out int32 [B*S, >= window + k] (row stride out.stride(0)), workspace a
    uint8 tensor of at least index_decode_workspace(B, S, N) bytes (the scores); flags: 0 or
    _lib.INDEX_EXACT (no effect: the scores are always the fixed-order ones)."""
    _on_gpu(q, keys, kscale, weights, nvis, pos, out, workspace)
    if out.dtype != torch.int32 or out.stride(-1) != 1:
        raise ValueError("out must be an int32 view with unit inner stride")
    B, S, Hi, Di = q.shape
    N = keys.shape[1]
    need = index_decode_workspace(B, S, N)
    if workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace holds {workspace.numel() * workspace.element_size()} bytes, needs {need}")
    if nvis is not None:
        nvis = nvis.to(torch.int32).contiguous()
    if pos is not None:
        pos = pos.to(torch.int32).contiguous()
    if kscale is not None:
        kscale = kscale.float().contiguous()
    q, keys, weights = q.contiguous(), keys.contiguous(), weights.float().contiguous()
    _lib.call("smla_index_decode", _p(q), dtype_code(q), _p(keys), dtype_code(keys), _p(kscale), _p(weights),
              _p(nvis), B, S, Hi, Di, N, k, _p(pos), window, _p(out), out.stride(0), int(id_offset), int(flags),
              _p(workspace), need, _stream(q))
    return out


def topk_into(scores, k, out, id_offset=0, nvis=None):
    """Write the top-k selection of scores [R, N] into the int32 view out [R, >=k] (row stride
    out.stride(0)); no allocation."""
    _on_gpu(scores, out, nvis)
    if out.dtype != torch.int32 or out.stride(-1) != 1:
        raise ValueError("out must be an int32 view with unit inner stride")
    R, N = scores.shape
    _lib.call("smla_topk", _p(scores), R, N, _p(nvis), k, _p(out), out.stride(0), int(id_offset),
              _stream(scores))
    return out
