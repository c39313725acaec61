"""ctypes binding of libsmla.so (the C ABI declared in include/smla.h).

The library is loaded from this directory.  There is no fallback: if the shared object is
missing or cannot be loaded, every op raises ``SmlaLibraryError``.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsmla.so")

F32, BF16, FP8_E4M3, F16, I32 = 0, 1, 2, 3, 4

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_int = ctypes.c_int
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes)
_SIGNATURES = {
    "smla_strerror": (ctypes.c_char_p, [_int]),
    "smla_api_version": (_int, []),
    "smla_sparse_attn": (_int, [_vp, _int, _vp, _i64, _vp, _i64, _int, _vp, _vp, _vp, _vp, _i64,
                                _i64, _i64, _i64, _i64, _i64, _f32, _vp, _int, _vp, _sz, _vp]),
    "smla_sparse_attn_workspace": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64, _int, _int]),
    "smla_sparse_attn_plan": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64, _int, _int, _int, _i64,
                                    ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "smla_sparse_attn_ex": (_int, [_vp, _int, _vp, _i64, _vp, _i64, _int, _vp, _vp, _vp, _vp, _i64,
                                   _i64, _i64, _i64, _i64, _i64, _f32, _vp, _int, _i64, _int, _vp, _sz, _vp]),
    "smla_sparse_attn_noalloc": (_int, [_vp, _int, _vp, _i64, _vp, _i64, _int, _vp, _vp, _vp, _vp, _i64,
                                        _i64, _i64, _i64, _i64, _i64, _f32, _vp, _int, _vp]),
    "smla_prefill_attn": (_int, [_vp, _int, _vp, _i64, _vp, _i64, _int, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                                 _i64, _i64, _f32, _vp, _int, _vp]),
    "smla_decode_attn_workspace": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _int, _int]),
    "smla_decode_attn": (_int, [_vp, _int, _vp, _i64, _vp, _i64, _int, _vp, _vp, _i64, _vp, _vp, _i64, _i64, _i64,
                                _i64, _i64, _i64, _i64, _f32, _vp, _int, _vp, _sz, _vp]),
    "smla_window_topk_idxs": (_int, [_i64, _i64, _i64, _i64, _vp, _vp]),
    "smla_decode_window_idxs": (_int, [_vp, _i64, _i64, _vp, _i64, _vp]),
    "smla_indexer_score": (_int, [_vp, _int, _vp, _int, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                  _vp, _vp]),
    "smla_indexer_score_fp4": (_int, [_vp, _int, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                      _vp, _vp]),
    "smla_topk": (_int, [_vp, _i64, _i64, _vp, _i64, _vp, _i64, _i32, _vp]),
    "smla_select_decode": (_int, [_vp, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i32, _vp]),
    "smla_index_decode": (_int, [_vp, _int, _vp, _int, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                                 _vp, _i64, _vp, _i64, _i32, _int, _vp, _sz, _vp]),
    "smla_index_decode_workspace": (_sz, [_i64, _i64, _i64]),
    "smla_block_mean_pool": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _vp, _int, _vp]),
    "smla_gated_pool": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _f32,
                               _int, _vp, _vp]),
    "smla_ring_step": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                              _f32, _int, _vp, _i64, _i64, _vp]),
    "smla_ring_step_kv": (_int, [_vp] * 9 + [_i64] * 5 + [_f32, _int, _vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp,
                                                           _i64, _i64, _f32, _int, _vp, _int, _i64, _vp]),
    "smla_quant_fp8_pow2": (_int, [_vp, _int, _i64, _i64, _vp, _vp, _vp]),
    "smla_row_epilogue": (_int, [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _int, _vp,
                                 _int, _i64, _vp]),
    "smla_row_epilogue_ids": (_int, [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _int, _vp,
                                     _int, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _vp]),
    "smla_decode_ids": (_int, [_vp, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _vp]),
    "smla_rotate_fp4": (_int, [_vp, _int, _i64, _i64, _int, _vp, _vp, _vp, _vp]),
    "smla_rope": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _int, _vp]),
    "smla_linear": (_int, [_vp, _int, _vp, _int, _i64, _i64, _i64, _i64, _vp, _int, _vp]),
    "smla_o_proj": (_int, [_vp, _int, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _int,
                           _i64, _vp, _vp, _int, _vp]),
}

# sim modes of smla_gated_pool / smla_ring_step, flags of smla_rotate_fp4
SIM_NONE, SIM_FP8, SIM_ROTATE_FP4 = 0, 1, 2
QAT_ROTATE, QAT_FP4 = 1, 2

# phases of smla_sparse_attn_ex, flags of smla_index_decode
ATTN_SPLIT, ATTN_MERGE = 1, 2
INDEX_EXACT = 1


class SmlaLibraryError(RuntimeError):
    """libsmla.so is missing or failed to load."""


class SmlaError(RuntimeError):
    """A libsmla entry point returned a non-zero status."""

    def __init__(self, fn, status, msg):
        super().__init__(f"{fn} failed with status {status}: {msg}")
        self.status = status


_LIB = None


def lib():
    """Load (once) and return the ctypes handle of libsmla.so."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise SmlaLibraryError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() (hipcc --offload-arch=gfx950)")
        try:
            handle = ctypes.CDLL(LIB_PATH)
        except OSError as e:  # pragma: no cover - depends on the machine
            raise SmlaLibraryError(f"cannot load {LIB_PATH}: {e}") from e
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def exported_symbols():
    return list(_SIGNATURES)


def check(fn_name, status):
    if status != 0:
        msg = lib().smla_strerror(status).decode()
        raise SmlaError(fn_name, status, msg)


def call(fn_name, *args):
    check(fn_name, getattr(lib(), fn_name)(*args))
