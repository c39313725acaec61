"""CPU tier: the C-ABI library loads, exports every symbol the header declares, maps status codes
and rejects bad arguments on the host before launching anything; the device fp8/bf16 codecs are
checked on the host against the oracle.  No compute call is made without a GPU."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest
import torch

from conftest import ROOT
from oracle import fp8

HEADER = os.path.join(ROOT, "include", "smla.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|size_t|const char\*)\s+(smla_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    from smla import _lib
    lib = _lib.lib()
    names = _declared()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.exported_symbols())
    assert lib.smla_api_version() == 2


def test_library_exports_only_declared_symbols():
    """`nm -D` of libsmla.so lists exactly the functions include/smla.h declares: no tuning hooks,
    no internal C++ symbols."""
    import shutil
    import subprocess
    from smla import _lib
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    res = subprocess.run([nm, "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    exported = {ln.split()[-1] for ln in res.stdout.splitlines() if len(ln.split()) >= 3 and ln.split()[1] in "TtWw"}
    assert exported == set(_declared()), (exported ^ set(_declared()))


def test_strerror_and_status_codes():
    from smla import _lib
    lib = _lib.lib()
    assert lib.smla_strerror(0) == b"ok"
    for code in range(-6, 0):
        assert lib.smla_strerror(code) and lib.smla_strerror(code) != b"unknown smla status"
    assert lib.smla_strerror(-99) == b"unknown smla status"


def test_host_validation_rejects_bad_arguments():
    from smla import _lib
    lib = _lib.lib()
    fake = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    # NULL inputs
    assert lib.smla_sparse_attn(None, 1, fake, 10, None, 0, 1, None, None, None, fake, 4, 1, 1, 64, 576, 512,
                                1.0, fake, 1, None, 0, None) == -1
    # DV > D
    assert lib.smla_sparse_attn(fake, 1, fake, 10, None, 0, 1, None, None, None, fake, 4, 1, 1, 64, 512, 576,
                                1.0, fake, 1, None, 0, None) == -2
    # second source without pointer
    assert lib.smla_sparse_attn(fake, 1, fake, 10, None, 5, 1, None, None, None, fake, 4, 1, 1, 64, 576, 512,
                                1.0, fake, 1, None, 0, None) == -1
    # bad dtype
    assert lib.smla_sparse_attn(fake, 9, fake, 10, None, 0, 1, None, None, None, fake, 4, 1, 1, 64, 576, 512,
                                1.0, fake, 1, None, 0, None) == -3
    # fp8 rows without scales
    assert lib.smla_sparse_attn(fake, 1, fake, 10, None, 0, 2, None, None, None, fake, 4, 1, 1, 64, 576, 512,
                                1.0, fake, 1, None, 0, None) == -1
    assert lib.smla_topk(fake, 2, 100, None, 10, fake, 5, 0, None) == -2        # stride < k
    assert lib.smla_topk(None, 2, 100, None, 10, fake, 10, 0, None) == -1
    assert lib.smla_topk(fake, 1, 70000, None, 10, fake, 10, 0, None) == -4     # N > 65536
    assert lib.smla_indexer_score(fake, 1, fake, 7, None, fake, None, 1, 1, 4, 64, 10, fake, None) == -3
    assert lib.smla_indexer_score(fake, 1, fake, 2, None, fake, None, 1, 1, 4, 48, 10, fake, None) == -4
    assert lib.smla_block_mean_pool(fake, 1, 1, 8, 12, 4, fake, 1, None) == -4   # D % 8
    assert lib.smla_gated_pool(fake, fake, fake, fake, fake, fake, 1, 8, 512, 4, 63, 1e-6, 0, fake, None) == -2
    assert lib.smla_gated_pool(fake, fake, fake, fake, fake, fake, 1, 8, 192, 4, 64, 1e-6, 0, fake, None) == -4
    assert lib.smla_gated_pool(fake, fake, fake, fake, fake, fake, 1, 8, 256, 4, 64, 1e-6, 3, fake, None) == -6
    odd = ctypes.c_void_p(4100)                                                  # kv/score/ape not 8-byte aligned
    assert lib.smla_gated_pool(odd, fake, fake, fake, fake, fake, 1, 8, 256, 4, 64, 1e-6, 0, fake, None) == -4
    assert lib.smla_gated_pool(fake, fake, odd, fake, fake, fake, 1, 8, 256, 4, 64, 1e-6, 0, fake, None) == -4
    ring_args = [fake] * 9 + [64, 2, 256, 4, 64, 1e-6, 0, fake, 8, 0, None]
    for i in (0, 2, 5):                                                          # ring_kv, kv_p, ape unaligned
        a = list(ring_args)
        a[i] = odd
        assert lib.smla_ring_step(*a) == -4
    a = list(ring_args)
    a[18] = 513                                                                  # odd projection row stride
    assert lib.smla_ring_step(*a) == -4
    # ring_step_kv: the ring's checks, the row epilogue's, and a window cache with rows
    rk = [fake] * 9 + [64, 2, 512, 4, 64, 1e-6, 0, fake, 8, 0]
    kv = [fake, 0, fake, fake, fake, 64, 64, 1e-6, 1, fake, 1, 64, None]
    assert lib.smla_ring_step_kv(*rk, *(kv[:11] + [0, None])) == -2             # kv_cache_rows 0
    assert lib.smla_ring_step_kv(*rk, *(kv[:8] + [2] + kv[9:])) == -4           # rotate-fp4 sim on the kv row
    assert lib.smla_ring_step_kv(*rk, *([None] + kv[1:])) == -1                 # kv_x missing
    assert lib.smla_ring_step_kv(*(rk[:18] + [1025]), *kv) == -4                # odd projection row stride
    # row_epilogue_ids: the row epilogue's checks, decode_ids', and rows of 512 only
    re = [fake, 64, 512, 0, 64, fake, None, fake, fake, 64, 64, 1e-6, 0, fake, 1, 0]
    di = [fake, 1, 128, 4, 1024, 256, fake, 384, None, None, 0, None]
    assert lib.smla_row_epilogue_ids(*(re[:2] + [256] + re[3:]), *di) == -4      # d 256
    assert lib.smla_row_epilogue_ids(*re, *(di[:2] + [0] + di[3:])) == -2       # window 0
    assert lib.smla_row_epilogue_ids(*re, *(di[:6] + [None] + di[7:])) == -1    # ids missing
    assert lib.smla_row_epilogue_ids(*(re[:12] + [2] + re[13:]), *di) == -4     # rotate-fp4 sim on q rows
    # rotate_fp4: row length, flags, codes without scales, dtype, alignment
    assert lib.smla_rotate_fp4(fake, 0, 4, 48, 3, fake, None, None, None) == -4
    assert lib.smla_rotate_fp4(fake, 0, 4, 2048, 3, fake, None, None, None) == -4
    assert lib.smla_rotate_fp4(fake, 0, 4, 64, 4, fake, None, None, None) == -4
    assert lib.smla_rotate_fp4(fake, 0, 4, 64, 3, None, fake, None, None) == -1
    assert lib.smla_rotate_fp4(fake, 0, 4, 64, 1, None, fake, fake, None) == -4     # codes need FP4
    assert lib.smla_rotate_fp4(fake, 0, 4, 64, 3, None, None, None, None) == -1     # no output
    assert lib.smla_rotate_fp4(fake, 2, 4, 64, 3, fake, None, None, None) == -3
    assert lib.smla_rotate_fp4(ctypes.c_void_p(24), 0, 4, 64, 3, fake, None, None, None) == -4
    assert lib.smla_rotate_fp4(fake, 0, 0, 64, 3, fake, None, None, None) == 0       # no rows
    assert lib.smla_quant_fp8_pow2(fake, 1, 4, 100, fake, fake, None) == -2
    assert lib.smla_window_topk_idxs(0, 1, 1, 0, fake, None) == -2
    assert lib.smla_decode_window_idxs(fake, 2, 128, fake, 64, None) == -2
    # row_epilogue: NULL, row width, rope without tables, sim, fp8 block, dtype, eps
    assert lib.smla_row_epilogue(None, 2, 512, 0, 1, None, None, None, None, 0, 0, 1e-6, 0, fake, 0, 0, None) == -1
    assert lib.smla_row_epilogue(fake, 2, 512, 256, 1, None, None, None, None, 0, 0, 1e-6, 0, fake, 0, 0, None) == -2
    assert lib.smla_row_epilogue(fake, 2, 96, 0, 1, None, None, None, None, 0, 0, 1e-6, 0, fake, 0, 0, None) == -2
    assert lib.smla_row_epilogue(fake, 2, 2048, 0, 1, None, None, None, None, 0, 0, 1e-6, 0, fake, 0, 0, None) == -2
    assert lib.smla_row_epilogue(fake, 2, 512, 0, 1, None, None, None, None, 0, 64, 1e-6, 0, fake, 0, 0, None) == -1
    assert lib.smla_row_epilogue(fake, 2, 512, 0, 1, None, None, None, None, 0, 0, 1e-6, 2, fake, 0, 0, None) == -4
    assert lib.smla_row_epilogue(fake, 2, 512, 0, 1, fake, None, fake, fake, 8, 32, 1e-6, 1, fake, 0, 0, None) == -2
    assert lib.smla_row_epilogue(fake, 2, 512, 0, 1, None, None, None, None, 0, 0, 1e-6, 0, fake, 9, 0, None) == -3
    assert lib.smla_row_epilogue(fake, 2, 512, 0, 1, None, None, None, None, 0, 0, -1.0, 0, fake, 0, 0, None) == -6
    assert lib.smla_row_epilogue(fake, 2, 512, 0, 1, None, None, None, None, 0, 0, 1e-6, 0, fake, 0, 16, None) == -1
    # decode_ids: NULL, T < window, only one of the compressed-row buffers, copy without ratio
    assert lib.smla_decode_ids(None, 2, 128, 4, 512, 16, fake, 144, None, None, 0, None) == -1
    assert lib.smla_decode_ids(fake, 2, 128, 4, 512, 16, fake, 100, None, None, 0, None) == -2
    assert lib.smla_decode_ids(fake, 2, 128, 4, 512, 16, fake, 144, fake, None, 512, None) == -1
    assert lib.smla_decode_ids(fake, 2, 128, 0, 512, 16, fake, 144, fake, fake, 512, None) == -2
    # a raw ring shorter than the window would alias its rows: decode_ids, select_decode
    assert lib.smla_decode_ids(fake, 2, 128, 4, 100, 16, fake, 144, None, None, 0, None) == -2
    assert lib.smla_select_decode(fake, 2, 1024, None, 64, fake, 128, fake, 192, 100, None) == -2


def _cpu_decode_layer():
    from smla import engine
    z = lambda *sh: torch.zeros(*sh, dtype=torch.bfloat16)
    w = engine.LayerWeights(wq_a=z(64, 512), q_a_norm=torch.ones(64), wq_b=z(64 * 512, 64), wkv=z(512, 512),
                            kv_a_norm=torch.ones(512), wo_a=z(8 * 16, 4096), wo_b=z(512, 128), sinks=torch.zeros(64))
    return engine.DecodeLayer(w, 1, ratio=0, max_pos=64, device="cpu")


def test_python_ops_refuse_cpu_tensors():
    from smla import compressor as sc
    from smla import mla
    from smla import norm_rope as snr
    from smla import qat as sq
    from smla import sparse_attn as ssa
    q = torch.zeros(1, 16, 576)
    kv = torch.zeros(8, 576)
    idx = torch.zeros(1, 4, dtype=torch.int32)
    with pytest.raises(Exception):
        ssa.sparse_attn(q, kv, None, idx, 1.0)
    # every mirror of the reference's functions refuses CPU tensors instead of running torch on them
    x = torch.zeros(2, 4096, dtype=torch.bfloat16)
    w = torch.zeros(1024, 4096, dtype=torch.bfloat16)
    cases = [
        lambda: mla.linear(x, w),
        lambda: mla.perhead_norm(torch.zeros(2, 64, 512)),
        lambda: mla.o_grouped(torch.zeros(2, 32768, dtype=torch.bfloat16), torch.zeros(8192, 4096), torch.zeros(4096, 8192)),
        lambda: snr.rmsnorm(torch.zeros(2, 8), torch.ones(8)),
        lambda: snr.apply_rotary_emb(torch.zeros(1, 4, 64), snr.precompute_freqs_cis(64, 4, 0, 1e4, 1, 32, 1)),
        lambda: sc.overlap_transform(torch.zeros(1, 2, 4, 16), 4, 8, 0.0),
        lambda: sc.compressor_prefill(torch.zeros(1, 8, 16), torch.zeros(256, 16), torch.zeros(256, 16),
                                      torch.zeros(4, 256), torch.ones(128), head_dim=128),
        lambda: sq.rotate_fp4(torch.zeros(4, 128)),
        lambda: _cpu_decode_layer(),
    ]
    for c in cases:
        with pytest.raises(RuntimeError):
            c()


@pytest.fixture(scope="module")
def codec(tmp_path_factory):
    out = tmp_path_factory.mktemp("codec") / "libcodec.so"
    src = os.path.join(ROOT, "tests", "native", "codec_host.hip")
    subprocess.run(["/opt/rocm/bin/hipcc", "-O2", "-fPIC", "-shared", "--offload-arch=gfx950", "-o", str(out), src],
                   check=True, capture_output=True)
    lib = ctypes.CDLL(str(out))
    lib.host_f32_to_e4m3.restype = ctypes.c_uint32
    lib.host_f32_to_e4m3.argtypes = [ctypes.c_float]
    lib.host_e4m3_to_f32.restype = ctypes.c_float
    lib.host_e4m3_to_f32.argtypes = [ctypes.c_uint32]
    lib.host_pow2_ceil.restype = ctypes.c_float
    lib.host_pow2_ceil.argtypes = [ctypes.c_float]
    lib.host_f32_to_bf16.restype = ctypes.c_uint16
    lib.host_f32_to_bf16.argtypes = [ctypes.c_float]
    lib.host_f32_to_e2m1.restype = ctypes.c_uint32
    lib.host_f32_to_e2m1.argtypes = [ctypes.c_float]
    lib.host_e2m1_to_f32.restype = ctypes.c_float
    lib.host_e2m1_to_f32.argtypes = [ctypes.c_uint32]
    lib.host_fp4_scale_exp.restype = ctypes.c_int
    lib.host_fp4_scale_exp.argtypes = [ctypes.c_float]
    lib.host_hadamard_scale.restype = ctypes.c_float
    lib.host_hadamard_scale.argtypes = [ctypes.c_int]
    return lib


def test_device_fp8_codec_matches_oracle(codec):
    codes = np.arange(256, dtype=np.uint8)
    ref = fp8.e4m3_decode(codes)
    for c in range(256):
        v = codec.host_e4m3_to_f32(c)
        assert (np.isnan(v) and np.isnan(ref[c])) or v == ref[c], c
    vals = ref[np.isfinite(ref)]
    pos = np.unique(np.abs(vals))
    mids = ((pos[1:].astype(np.float64) + pos[:-1]) / 2).astype(np.float32)
    rng = np.random.default_rng(3)
    rnd = np.clip(rng.standard_normal(4000).astype(np.float32) * 50, -448, 448)
    x = np.concatenate([vals, mids, -mids, np.nextafter(mids, 0), np.nextafter(mids, 1), rnd,
                        np.float32([2.0 ** -10, 3 * 2.0 ** -10, 1e-30, -0.0])])
    want = fp8.e4m3_encode(x)
    got = np.array([codec.host_f32_to_e4m3(float(v)) for v in x], dtype=np.uint32)
    np.testing.assert_array_equal(got, want.astype(np.uint32))


def test_device_pow2_and_bf16_match_oracle(codec):
    rng = np.random.default_rng(4)
    amax = np.concatenate([np.exp2(rng.uniform(-13, 12, 500)), np.exp2(np.arange(-13, 12)) * 448.0]).astype(np.float32)
    e = fp8.pow2_scale_exponent(amax)
    for a, ee in zip(amax, e):
        assert codec.host_pow2_ceil(float(np.float32(a / np.float32(448.0)))) == 2.0 ** ee
    x = rng.standard_normal(2000).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([codec.host_f32_to_bf16(float(v)) for v in x], dtype=np.uint16)
    np.testing.assert_array_equal(got, ref)


def test_device_fp4_codec_matches_oracle(codec):
    from oracle import qat
    for c in range(16):
        v = codec.host_e2m1_to_f32(c)
        assert v == qat.e2m1_value(c) and np.signbit(v) == bool(c & 8), c
    grid = qat.FP4_GRID.astype(np.float64)
    mids = ((grid[1:] + grid[:-1]) / 2).astype(np.float32)
    rng = np.random.default_rng(5)
    x = np.concatenate([qat.FP4_GRID, mids, np.nextafter(mids, 0), np.nextafter(mids, 7),
                        rng.uniform(-6, 6, 3000).astype(np.float32)])
    x = np.concatenate([x, -x, np.float32([-0.0, 1e-30, -1e-30])]).astype(np.float32)
    got = np.array([codec.host_f32_to_e2m1(float(v)) for v in x], dtype=np.uint8)
    np.testing.assert_array_equal(got, qat.e2m1_code(x))
    amax = np.concatenate([(rng.uniform(0.5, 1, 2000) * np.exp2(rng.integers(-140, 120, 2000))),
                           6.0 * np.exp2(np.arange(-126.0, 126.0)), [0.0, 3.4e38]]).astype(np.float32)
    got = np.array([codec.host_fp4_scale_exp(float(a)) for a in amax])
    np.testing.assert_array_equal(got, qat.fp4_scale_exponent(amax))
    for lg in range(5, 11):
        assert codec.host_hadamard_scale(lg) == qat.rotate_scale(2 ** lg)


def test_layer_wrappers_check_sizes():
    """The fused layer wrappers check the extents the C entries cannot see before anything reaches a
    kernel: one position per sequence, norm weights per channel, table width, room in out (rows or
    the cache), the ids and emitted-row buffers, and ring_step_kv's position count and cache rows.
    The checks come before the device check, so CPU tensors show them."""
    from smla import _lib, ops
    x = torch.zeros(4, 512)
    out = torch.zeros(4, 512)
    pos = torch.zeros(4, dtype=torch.int32)
    cs = torch.zeros(64, 32)
    re = lambda **kw: ops.row_epilogue(**{**dict(x=x, norm_w=None, pos=pos, cos_t=cs, sin_t=cs, rd=64,
                                                 sim=_lib.SIM_NONE, out=out), **kw})
    with pytest.raises(ValueError, match="positions"):
        re(pos=torch.zeros(3, dtype=torch.int32))                        # pos count != rows
    with pytest.raises(ValueError, match="whole number"):
        re(rows_per_pos=3)                                               # 4 rows, 3 per position
    with pytest.raises(ValueError, match="norm_w"):
        re(norm_w=torch.ones(256))
    with pytest.raises(ValueError, match="tables"):
        re(cos_t=torch.zeros(64, 16), sin_t=torch.zeros(64, 16))
    with pytest.raises(ValueError, match="out holds"):
        re(out=torch.zeros(3, 512))                                      # too few rows
    with pytest.raises(ValueError, match="out holds"):
        re(out=torch.zeros(4, 8, 512), cache_rows=16)                    # cache of 8 rows, 16 claimed
    with pytest.raises(ValueError, match="need positions"):
        re(pos=None)
    # decode_ids: ids shape, emitted-row buffers
    ids_pos = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="ids must be"):
        ops.decode_ids(ids_pos, 128, 4, 128, 16, 144, out=torch.zeros(2, 100, dtype=torch.int32))
    with pytest.raises(ValueError, match="comp32 / comp_out"):
        ops.decode_ids(ids_pos, 128, 4, 128, 16, 144, comp32=torch.zeros(2, 8, 512),
                       comp_out=torch.zeros(2, 8, 512, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="go together"):
        ops.decode_ids(ids_pos, 128, 4, 128, 16, 144, comp32=torch.zeros(2, 16, 512))
    # row_epilogue_ids: both sets of checks
    with pytest.raises(ValueError, match="ids must be"):
        ops.row_epilogue_ids(x, None, ids_pos, cs, cs, 64, _lib.SIM_NONE, out, 2, ids_pos, 128, 4, 128, 16, 144,
                             torch.zeros(2, 128, dtype=torch.int32))
    with pytest.raises(ValueError, match="positions"):
        ops.row_epilogue_ids(x, None, pos[:3], cs, cs, 64, _lib.SIM_NONE, out, 1, ids_pos, 128, 4, 128, 16, 144,
                             torch.zeros(2, 144, dtype=torch.int32))

    # ring_step_kv: one position per sequence, cache rows within the cache
    class _Ring:
        ring_kv = torch.zeros(2, 8, 1024)
    with pytest.raises(ValueError, match="positions"):
        ops.ring_step_kv(_Ring, None, None, torch.zeros(3, dtype=torch.int32), None, None, None, None, None, 64,
                         _lib.SIM_FP8, torch.zeros(2, 128, 512))
    with pytest.raises(ValueError, match="cache_rows"):
        ops.ring_step_kv(_Ring, None, None, torch.zeros(2, dtype=torch.int32), None, None, None, None, None, 64,
                         _lib.SIM_FP8, torch.zeros(2, 128, 512), cache_rows=256)
