"""Indexer-key transform with the signatures of ``v4mlx/qat.py``, on the GPU.

* ``hadamard_rotate(x)`` — ``v4mlx/qat.py:8-20``: normalised Walsh-Hadamard (Sylvester order) over
  the last dim, float32 butterfly, times float32(n ** -0.5).
* ``fp4_act_quant(x, block=32)`` — ``v4mlx/qat.py:23-31``: per-32 pow2-scaled fp4 e2m1 round trip.
* ``rotate_fp4(x)`` — both, in one pass: the indexer compressor's key transform
  (``v4mlx/compressor.py:57-59``).
* ``fp4_pack(x, rotate=True)`` — the stored form of the same result: packed e2m1 codes
  ``[..., n/2]`` (element 2i in the low nibble) and ue8m0 scales ``[..., n/32]`` (log2(s) + 127).

All four run one HIP kernel (``smla_rotate_fp4``); the last dim must be a power of two in
32..1024.  Results are float32 (the reference returns float32 arrays)."""
from . import ops


def hadamard_rotate(x):
    return ops.rotate_fp4_op(x, True, False, True, False)[0]


def fp4_act_quant(x, block=32):
    if block != 32:
        raise ValueError("fp4_act_quant: the kernel quantises blocks of 32")
    return ops.rotate_fp4_op(x, False, True, True, False)[0]


def rotate_fp4(x):
    return ops.rotate_fp4_op(x, True, True, True, False)[0]


def fp4_pack(x, rotate=True):
    _, codes, scales = ops.rotate_fp4_op(x, bool(rotate), True, False, True)
    return codes, scales
