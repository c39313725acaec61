"""Indexer scoring and stable top-k selection (CPU oracle).

The reference has NO indexer and NO score-based top-k: its engine attends every causally visible
compressed row (``oracle/decode_engine.py:110-114``).  The indexer here is the build's own
definition, following the public DeepSeek sparse-attention design (ReLU-gated per-head dot
products, per-head weights, per-key scale), with one fixed fp32 arithmetic order so that GPU and
CPU agree bit for bit (``indexer_ref.c`` spells it out).  Selection ranks visible positions by
(score descending, index ascending), -0 == +0, keeps min(k, nvis), returns them ascending,
-1 padded.  When nvis <= k the selection is "all visible rows", i.e. exactly the reference's
index build.

Pinning: ``score_bruteforce`` recomputes the chain with exact rational arithmetic rounded to
float32 after every fused step (Python ``fractions``) on tiny inputs; ``topk_bruteforce`` is a
Python sort with the same tie rule; the nvis <= k case is compared with the reference's closed
form.  Beyond that the definition is the build's, so "bit-exact" means bit-exact to this chain.
"""
import ctypes
import os
from fractions import Fraction

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle_smla.so")
        if not os.path.exists(path):
            import subprocess
            subprocess.run(["make", "-s", "-C", _HERE], check=True)
        lib = ctypes.CDLL(path)
        f32p = ctypes.POINTER(ctypes.c_float)
        i32p = ctypes.POINTER(ctypes.c_int32)
        i64 = ctypes.c_int64
        lib.oracle_indexer_score.argtypes = [f32p, f32p, f32p, f32p, i64, i64, i64, i64, i32p, f32p]
        lib.oracle_indexer_score.restype = None
        lib.oracle_topk.argtypes = [f32p, i64, i64, i32p, i64, i32p]
        lib.oracle_topk.restype = None
        _LIB = lib
    return _LIB


def _fp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)) if a is not None else None


def _ip(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)) if a is not None else None


def indexer_score(q, k, kscale, w, nvis=None):
    """q:[S,H,D] fp32, k:[N,D] fp32, kscale:[N] fp32 or None, w:[S,H] fp32, nvis:[S] int or None
    -> scores [S,N] fp32 (positions >= nvis are -inf)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    ks = None if kscale is None else np.ascontiguousarray(kscale, dtype=np.float32)
    nv = None if nvis is None else np.ascontiguousarray(nvis, dtype=np.int32)
    S, H, D = q.shape
    N = k.shape[0]
    out = np.empty((S, N), dtype=np.float32)
    _lib().oracle_indexer_score(_fp(q), _fp(k), _fp(ks), _fp(w), S, H, D, N, _ip(nv), _fp(out))
    return out


def topk(scores, k, nvis=None):
    """scores:[R,N] fp32 -> [R,k] int32 ascending selected ids, -1 padded."""
    s = np.ascontiguousarray(scores, dtype=np.float32)
    R, N = s.shape
    nv = None if nvis is None else np.ascontiguousarray(nvis, dtype=np.int32)
    out = np.empty((R, k), dtype=np.int32)
    _lib().oracle_topk(_fp(s), R, N, _ip(nv), k, _ip(out))
    return out


def _round_f32(x: Fraction) -> Fraction:
    """Round an exact rational to the nearest float32 (ties to even)."""
    return Fraction(float(np.float32(_nearest_f64_then_check(x))))


def _nearest_f64_then_check(x: Fraction):
    # Exact rounding to float32: find the float32 neighbours around x and pick by distance.
    f = np.float32(float(x))                       # may be off by one ulp through double rounding
    cands = [f, np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(-np.inf))]
    best = None
    for c in cands:
        if not np.isfinite(c):
            continue
        dist = abs(Fraction(float(c)) - x)
        if best is None or dist < best[0] or (dist == best[0] and (int(np.float32(c).view(np.uint32)) & 1) == 0):
            best = (dist, c)
    return best[1]


def score_bruteforce(q, k, kscale, w, nvis=None):
    """Exact-rational restatement of the chain (tiny inputs only)."""
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    w = np.asarray(w, dtype=np.float32)
    S, H, D = q.shape
    N = k.shape[0]
    out = np.empty((S, N), dtype=np.float32)
    for s in range(S):
        nv = N if nvis is None else int(nvis[s])
        for n in range(N):
            if n >= nv:
                out[s, n] = -np.inf
                continue
            acc = Fraction(0)
            for h in range(H):
                dot = Fraction(0)
                for d in range(D):
                    dot = _round_f32(Fraction(float(q[s, h, d])) * Fraction(float(k[n, d])) + dot)
                r = dot if dot > 0 else Fraction(0)
                acc = _round_f32(Fraction(float(w[s, h])) * r + acc)
            val = np.float32(float(acc))
            if kscale is not None:
                val = np.float32(val * np.float32(kscale[n]))
            out[s, n] = val
    return out


def topk_bruteforce(scores, k, nvis=None):
    R, N = scores.shape
    out = np.full((R, k), -1, dtype=np.int32)
    for r in range(R):
        nv = N if nvis is None else int(nvis[r])
        items = [(-(float(scores[r, n]) + 0.0), n) for n in range(nv)]
        items.sort()
        sel = sorted(n for _, n in items[:k])
        out[r, : len(sel)] = sel
    return out
