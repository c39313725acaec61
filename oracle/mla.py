"""Grouped low-rank output projection and plain linear of the MLA block (CPU oracle).

Restates:

* ``linear``     — ``v4mlx/mla.py:16-18``: y = x @ W^T, here in float64;
* ``o_grouped``  — ``v4mlx/mla.py:42-56``: o [T, heads*head_dim] split into G equal slices
  (slice g = heads g*H/G .. (g+1)*H/G - 1); slice g times wo_a's rows g*R .. (g+1)*R - 1
  (transposed) gives mid[:, g*R:(g+1)*R]; y = mid @ wo_b^T.  Products and sums in float64; the
  intermediate ``mid`` is rounded to bfloat16 when ``mid_bf16`` (the dtype the decode path keeps
  it in), else kept in float64;
* ``o_project``  — ``oracle/decode_engine.py:118-119``: the inverse RoPE of the last rd dims of
  every head (``norm_rope.apply_rotary_emb`` with ``inverse=True``, float32, rounded back to o's
  dtype), then ``o_grouped``.

Pinning (``tests/test_oracle_mla.py``): ``o_grouped`` equals o @ blockdiag(wa_0^T, ..., wa_{G-1}^T)
@ wo_b^T built with ``scipy.linalg.block_diag`` (a library routine), and its G = 1 case is the
plain product; ``o_project`` at position 0 (cos 1, sin 0) is ``o_grouped`` of o itself, and a
rotation by a quarter turn swaps each rope pair.
"""
import numpy as np
import torch

from .norm_rope import apply_rotary_emb


def linear(x, W):
    return np.asarray(x, dtype=np.float64) @ np.asarray(W, dtype=np.float64).T


def _bf16(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(torch.bfloat16).float().numpy().astype(np.float64)


def o_grouped(o, wo_a, wo_b, groups=8, mid_bf16=True):
    o = np.asarray(o, dtype=np.float64)
    wa = np.asarray(wo_a, dtype=np.float64)
    T, HD = o.shape
    K = HD // groups
    R = wa.shape[0] // groups
    mid = np.concatenate([o[:, g * K:(g + 1) * K] @ wa[g * R:(g + 1) * R].T for g in range(groups)], axis=1)
    if mid_bf16:
        mid = _bf16(mid)
    return mid @ np.asarray(wo_b, dtype=np.float64).T


def o_project(o, pos, cos_t, sin_t, wo_a, wo_b, groups=8, mid_bf16=True):
    """o: torch [T, heads, head_dim] (bf16 or fp32); pos [T]; cos_t/sin_t [n_pos, rd/2] fp32."""
    T, H, D = o.shape
    rd = 2 * cos_t.shape[1]
    cis = torch.complex(cos_t[pos.long()], sin_t[pos.long()])          # [T, rd/2]
    rot = apply_rotary_emb(o[None, :, :, D - rd:], cis, inverse=True)[0]
    o2 = torch.cat([o[..., :D - rd], rot], dim=-1)
    return o_grouped(o2.float().reshape(T, H * D).numpy(), wo_a, wo_b, groups, mid_bf16)
