"""GPU check of smla_sparse_attn_noalloc, the allocation-free variant of smla_sparse_attn: called
through the C ABI, its output equals smla_sparse_attn's (same plan and kernels, workspace given)
bit for bit on two calls in a row, the second smaller than the first, and both are within the bf16
tolerance of the oracle.  A plan whose partial states exceed the library's buffer is refused with
SMLA_E_WORKSPACE before anything runs."""

import pytest
import torch

from conftest import announce
from oracle import sparse_attn as osa

pytestmark = pytest.mark.gpu

BF16_ABS, BF16_REL = 2e-2, 1e-2


def _inputs(B, H, n0, n1, T, seed):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, 1, H, 576, generator=g) * 0.05).to(torch.bfloat16)
    kv0 = (torch.randn(B, n0, 576, generator=g) * 0.5).to(torch.bfloat16)
    kv1 = (torch.randn(B, n1, 576, generator=g) * 0.5).to(torch.bfloat16)
    idx = torch.randint(0, n0 + n1, (B, 1, T), generator=g, dtype=torch.int32)
    idx[..., -3:] = -1
    sink = torch.randn(H, generator=g)
    return q, kv0, kv1, idx, sink


def _call(fn, q, kv0, kv1, idx, sink, out, out_dtype, ws=None):
    from smla import _lib
    lib = _lib.lib()
    B, S, H, D = q.shape
    T = idx.shape[-1]
    args = [q.data_ptr(), _lib.BF16, kv0.data_ptr(), kv0.shape[1], kv1.data_ptr(), kv1.shape[1], _lib.BF16, None,
            None, sink.data_ptr(), idx.data_ptr(), T, B, S, H, D, 512, 576 ** -0.5, out.data_ptr(), out_dtype]
    if fn == "smla_sparse_attn":
        args += [ws.data_ptr(), ws.numel()]
    return getattr(lib, fn)(*args, None)


def test_noalloc_matches_workspace_path(dev):
    from smla import _lib, ops
    for step, (B, H, n0, n1, T, seed) in enumerate([(8, 64, 4000, 2000, 2176, 1), (2, 64, 500, 300, 300, 2)]):
        announce(f"noalloc call {step}: B={B} H={H} T={T}")
        q, kv0, kv1, idx, sink = [t.to(dev) for t in _inputs(B, H, n0, n1, T, seed)]
        ns, _, wsb = ops.attn_plan(B, 1, H, 576, 512, T)
        assert wsb <= 32 << 20
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        want = torch.empty(B, 1, H, 512, dtype=torch.bfloat16, device=dev)
        got = torch.full_like(want, float("nan"))
        assert _call("smla_sparse_attn", q, kv0, kv1, idx, sink, want, _lib.BF16, ws) == 0
        assert _call("smla_sparse_attn_noalloc", q, kv0, kv1, idx, sink, got, _lib.BF16) == 0
        torch.cuda.synchronize()
        assert ns > 1, ns                      # the partial states went through the buffer
        assert torch.equal(got, want), f"call {step}: differs from the workspace path"
        kv = [torch.cat([kv0[b].float(), kv1[b].float()]).cpu() for b in range(B)]
        for b in range(B):
            ref = osa.sparse_attn(q[b].float().cpu(), kv[b], sink.cpu(), idx[b].long().cpu(), 576 ** -0.5, dv=512)
            o = got[b].float().cpu()
            err = (o - ref).abs().max().item()
            assert err <= BF16_ABS and err / ref.abs().max().item() <= BF16_REL, f"call {step} seq {b}: {err:.3e}"


def test_noalloc_refuses_plans_beyond_its_buffer(dev):
    """128 sequences of 256 ids with fp32 output: two splits each, 33.7 MB of fp32 partial states
    against the 32 MiB buffer."""
    from smla import _lib, ops
    announce("noalloc refuses a plan beyond its buffer")
    B, H, T = 128, 64, 256
    ns, _, wsb = ops.attn_plan(B, 1, H, 576, 512, T, out_dtype=torch.float32)
    assert wsb > 32 << 20, (ns, wsb)
    q, kv0, kv1, idx, sink = [t.to(dev) for t in _inputs(B, H, 300, 100, T, 3)]
    out = torch.zeros(B, 1, H, 512, dtype=torch.float32, device=dev)
    assert _call("smla_sparse_attn_noalloc", q, kv0, kv1, idx, sink, out, _lib.F32) == -5   # SMLA_E_WORKSPACE
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0       # nothing ran
