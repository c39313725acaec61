"""smla — MI355X (gfx950) sparse multi-head latent attention for DeepSeek-V4-Flash.

Drop-in replacements for the reference's hot-path functions, backed by hand-written HIP kernels
in libsmla.so (C ABI: include/smla.h):

* ``smla.sparse_attn``  — ``ref_torch/sparse_attn.py`` (``sparse_attn``, ``get_window_topk_idxs``)
* ``smla.compressor``   — ``ref_torch/compressor.py`` (``overlap_transform``, ``compressor_prefill``)
                          plus block mean pooling and the device-resident decode ring
* ``smla.indexer``      — indexer scoring and exact top-k selection
* ``smla.norm_rope``    — ``ref_torch/norm_rope.py`` (tables for the kernels)
* ``smla.mla``          — ``v4mlx/mla.py`` projections
* ``smla.workloads``    — seeded synthetic inputs of the benchmark configurations
"""
from . import _lib  # noqa: F401
from ._lib import SmlaError, SmlaLibraryError  # noqa: F401


def load():
    """Load libsmla.so now (raises SmlaLibraryError if it is missing)."""
    return _lib.lib()
