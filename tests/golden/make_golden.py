"""Writes the golden fixtures under tests/golden/ by running the reference's torch functions.

Run in the build container only (the reference is not present on GPU machines):

    python tests/golden/make_golden.py

Only functions whose exact fp32 results no closed form or library routine fixes are run here:
``ref_torch/compressor.py`` (``overlap_transform``, ``compressor_prefill`` with its state dict)
and ``ref_torch/norm_rope.py`` (``precompute_freqs_cis`` table rounding, ``apply_rotary_emb``,
``rmsnorm``).  Inputs are seeded; the fixtures hold inputs and outputs as plain arrays (.npz,
no pickles).
"""
import os
import sys

import numpy as np
import torch

REF = "/root/reference"
OUT = os.path.dirname(os.path.abspath(__file__))


def main():
    sys.path.insert(0, REF)
    from ref_torch import compressor as rc          # noqa: E402
    from ref_torch import norm_rope as rn           # noqa: E402

    g = torch.Generator().manual_seed(1234)

    # --- RoPE tables and rotation ---------------------------------------------------------
    fy = rn.precompute_freqs_cis(64, 96, 65536, 160000.0, 16, 32, 1)
    fn = rn.precompute_freqs_cis(64, 96, 0, 10000.0, 40, 32, 1)
    x3 = torch.randn(1, 96, 64, generator=g)
    x4 = torch.randn(1, 96, 2, 64, generator=g)
    np.savez(os.path.join(OUT, "norm_rope.npz"),
             freqs_yarn_re=fy.real.numpy(), freqs_yarn_im=fy.imag.numpy(),
             freqs_plain_re=fn.real.numpy(), freqs_plain_im=fn.imag.numpy(),
             x3=x3.numpy(), x4=x4.numpy(),
             rope3=rn.apply_rotary_emb(x3, fy).numpy(),
             rope3_inv=rn.apply_rotary_emb(x3, fy, inverse=True).numpy(),
             rope4=rn.apply_rotary_emb(x4, fy).numpy(),
             rms_x=x3[0, :16].numpy(), rms_w=torch.linspace(0.5, 1.5, 64).numpy(),
             rms_out=rn.rmsnorm(x3[0, :16], torch.linspace(0.5, 1.5, 64)).numpy())

    # --- overlap transform -----------------------------------------------------------------
    t = torch.randn(2, 3, 4, 16, generator=g)
    np.savez(os.path.join(OUT, "overlap.npz"), t=t.numpy(),
             zero=rc.overlap_transform(t, 4, 8, 0).numpy(),
             ninf=rc.overlap_transform(t, 4, 8, float("-inf")).numpy())

    # --- compressor prefill: small and model-width heads, with and without remainder -------
    cases = {}
    for name, (b, s, dim, d, rd) in {"small_rem": (2, 18, 32, 16, 4),
                                     "small_even": (1, 16, 32, 16, 4),
                                     "wide_rem": (1, 37, 24, 512, 64)}.items():
        x = torch.randn(b, s, dim, generator=g)
        wkv = torch.randn(2 * d, dim, generator=g) * dim ** -0.5
        wgate = torch.randn(2 * d, dim, generator=g) * dim ** -0.5
        ape = torch.randn(4, 2 * d, generator=g) * 0.5
        norm_w = 1 + 0.1 * torch.randn(d, generator=g)
        kv, state = rc.compressor_prefill(x, wkv, wgate, ape, norm_w, head_dim=d, ratio=4, rope_head_dim=rd)
        entry = dict(x=x, wkv=wkv, wgate=wgate, ape=ape, norm_w=norm_w, kv=kv)
        for key, val in state.items():
            entry["state_" + key] = val
        for key, val in entry.items():
            cases[f"{name}__{key}"] = val.numpy()
        cases[f"{name}__dims"] = np.array([b, s, dim, d, rd])
    np.savez(os.path.join(OUT, "compressor.npz"), **cases)
    print("wrote", sorted(os.listdir(OUT)))


if __name__ == "__main__":
    main()
