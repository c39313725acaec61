"""CPU tier: the attention op's operand checks raise ValueError before any launch (a mismatch would
send the kernel's row, index or scale addressing past its buffers)."""
import pytest
import torch


def _ops():
    from smla import ops
    return ops


def _ok():
    B, S, H, D = 2, 3, 64, 576
    return dict(q=torch.empty(B, S, H, D, dtype=torch.bfloat16), kv0=torch.empty(B, 100, D, dtype=torch.bfloat16),
                kv1=torch.empty(B, 40, D, dtype=torch.bfloat16), kv0_scale=None, kv1_scale=None,
                attn_sink=torch.empty(H), topk_idxs=torch.empty(B, S, 7, dtype=torch.int32), dv=512)


def test_matching_operands_pass():
    _ops()._check_attn(**_ok())


@pytest.mark.parametrize("change", [
    dict(kv0=torch.empty(3, 100, 576, dtype=torch.bfloat16)),          # batch differs from q's
    dict(kv0=torch.empty(2, 100, 512, dtype=torch.bfloat16)),          # row width differs from D
    dict(kv1=torch.empty(2, 40, 512, dtype=torch.bfloat16)),
    dict(kv1=torch.empty(1, 40, 576, dtype=torch.bfloat16)),
    dict(kv1=torch.empty(2, 40, 576, dtype=torch.float32)),            # kv1 dtype differs from kv0's
    dict(topk_idxs=torch.empty(2, 1, 7, dtype=torch.int32)),           # [B,1,T] with S=3
    dict(topk_idxs=torch.empty(2, 3, dtype=torch.int32)),
    dict(attn_sink=torch.empty(32)),
    dict(dv=577),
    dict(dv=0),
    dict(kv0_scale=torch.empty(2, 100, 9)),                            # scales for bf16 rows
])
def test_mismatches_raise(change):
    args = _ok()
    args.update(change)
    with pytest.raises(ValueError):
        _ops()._check_attn(**args)


def test_fp8_scale_shapes():
    ops = _ops()
    args = _ok()
    args.update(kv0=torch.empty(2, 100, 576, dtype=torch.uint8), kv1=torch.empty(2, 40, 576, dtype=torch.uint8),
                kv0_scale=torch.empty(2, 100, 9), kv1_scale=torch.empty(2, 40, 9))
    ops._check_attn(**args)
    for bad in (dict(kv0_scale=None), dict(kv1_scale=torch.empty(2, 41, 9)), dict(kv0_scale=torch.empty(2, 100, 8)),
                dict(kv1_scale=torch.empty(2, 40, 9, dtype=torch.float16))):
        a = dict(args)
        a.update(bad)
        with pytest.raises(ValueError):
            ops._check_attn(**a)
