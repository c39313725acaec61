"""CPU oracle for the sparse-MLA attention path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes on the hot path, so that the
HIP kernels can be checked against it on identical inputs.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only
as the checker (or the timed CPU baseline) — never as the product path.  The product path
(``deepseek-v4-flash-mlx_amd/smla``) never imports this package and fails loudly when its HIP
library is missing.

Modules and the reference functions they restate:

* ``norm_rope``   — ``ref_torch/norm_rope.py`` (RMSNorm, YaRN frequencies, interleaved RoPE).
* ``fp8``         — e4m3fn round-to-nearest-even encode/decode and the pow2-scale block
                    act-quant of ``v4mlx/compressor.py:11-20`` / ``oracle/decode_engine.py:52-54``.
* ``sparse_attn`` — ``ref_torch/sparse_attn.py`` (window indices, dense-gather sparse attention)
                    and the engine's index build ``oracle/decode_engine.py:107-114``.
* ``compressor``  — ``ref_torch/compressor.py`` (overlap transform, gated pooling prefill), the
                    decode ring step ``oracle/decode_engine.py:96-105`` and block mean pooling.
* ``indexer``     — indexer scoring and stable top-k selection.  The reference has no indexer;
                    the definition is the build's own (see the module docstring).  The
                    canonical fp32 score chain runs in plain C (``indexer_ref.c``) so that the
                    fused-multiply-add rounding is exact.
* ``qat``         — Walsh–Hadamard rotation and fp4 block quantisation of ``v4mlx/qat.py``.

How each function is pinned (golden vectors, closed forms, library routines, brute force) is
recorded in each module's header.  A function without such a check says "parity unpinned".
"""
