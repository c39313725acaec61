"""The error bound of the certified MFMA indexer path, checked on the CPU against the oracle.

indexer_cert_kernel (csrc/indexer.hip) bounds the distance between its approximate score a_n and
the fixed-order score s_n by
    e_n = (|ks| (2^-15 W1 + 2^-14 PW + 2^-100 (|w|_1 + 1)) + 2^-22 |a_n| + 2^-126) (1 + 2^-10),
W1 = sum_h |w_h| ReLU(dot_h), PW = sum_h |w_h| P_h with P_h = sum_d |q_hd k_d| as the MFMA computes
it, and the selection's correctness rests on |a_n - s_n| <= e_n.  Three models of the MFMA
arithmetic stand in for the hardware: every dot product exact and rounded once; fp32 sums in
reverse order with the head sums in another order; and products below 2^-126 flushed to zero
(in the dot products and in P alike).  The fixed-order score comes from the oracle.

The bound must hold with a factor 3 to spare.  The inputs are built so that the bound's terms are
needed: small products added to large cancelling partial sums (the fixed-order chain loses most of
them: only the PW term covers that), and products in the subnormal range under the flushing model
(only the absolute term covers those).  Each such case also checks that the bound without its
term fails, so a dropped term cannot pass unnoticed."""
import numpy as np
import pytest

from oracle import indexer as oidx


def _bf16(x):
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32)


def _e4m3_grid():
    vals = []
    for c in range(256):
        s, e, m = (c >> 7) & 1, (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            continue
        v = m * 2.0 ** -9 if e == 0 else 2.0 ** (e - 7) * (1 + m / 8)
        vals.append(-v if s else v)
    return np.array(vals, dtype=np.float32)


def _bound(a, ks, w, dots, P, use_pw=True, use_tiny=True):
    aw = np.abs(w).astype(np.float64)
    W1 = (aw[None, :] * np.maximum(dots, 0)).sum(1)
    PW = (aw[None, :] * P).sum(1) if use_pw else 0.0
    wn1 = aw.sum()
    tiny = 2.0 ** -100 * (wn1 + 1) if use_tiny else 0.0
    return (np.abs(ks) * (2.0 ** -15 * W1 + 2.0 ** -14 * PW + tiny) + 2.0 ** -22 * np.abs(a)
            + (2.0 ** -126 if use_tiny else 0.0)) * (1 + 2.0 ** -10)


def _model_exact_round(q, k, w, ks):
    q64, k64 = q.astype(np.float64), k.astype(np.float64)
    dots = (k64 @ q64.T).astype(np.float32)
    P = (np.abs(k64) @ np.abs(q64).T).astype(np.float32)
    acc = (np.maximum(dots, 0).astype(np.float64) * w[None, :]).sum(1).astype(np.float32)
    return (acc * ks).astype(np.float32), dots.astype(np.float64), P.astype(np.float64)


def _model_reverse_f32(q, k, w, ks):
    N, D = k.shape
    dots = np.zeros((N, q.shape[0]), dtype=np.float32)
    P = np.zeros((N, q.shape[0]), dtype=np.float32)
    for d in reversed(range(D)):
        prod = np.outer(k[:, d], q[:, d]).astype(np.float32)
        dots = (dots + prod).astype(np.float32)
        P = (P + np.abs(prod)).astype(np.float32)
    r = np.maximum(dots, 0)
    acc = np.zeros(N, dtype=np.float32)
    for h in [*range(1, q.shape[0], 2), *range(0, q.shape[0], 2)]:
        acc = (acc + (r[:, h] * w[h]).astype(np.float32)).astype(np.float32)
    return (acc * ks).astype(np.float32), dots.astype(np.float64), P.astype(np.float64)


def _model_ftz(q, k, w, ks):
    prod = k.astype(np.float64)[:, None, :] * q.astype(np.float64)[None, :, :]   # [N, H, D]
    prod = np.where(np.abs(prod) < 2.0 ** -126, 0.0, prod)
    dots = prod.sum(2).astype(np.float32)
    P = np.abs(prod).sum(2).astype(np.float32)
    acc = (np.maximum(dots, 0).astype(np.float64) * w[None, :]).sum(1).astype(np.float32)
    return (acc * ks).astype(np.float32), dots.astype(np.float64), P.astype(np.float64)


MODELS = [_model_exact_round, _model_reverse_f32, _model_ftz]


def _inputs(case, rng):
    grid = _e4m3_grid()
    H = D = 64
    N = 1024
    q = _bf16(rng.standard_normal((H, D)).astype(np.float32))
    k = rng.choice(grid[np.abs(grid) <= 4], size=(N, D)).astype(np.float32)
    ks = (2.0 ** rng.integers(-8, 4, N)).astype(np.float32)
    w = rng.standard_normal(H).astype(np.float32)
    if case == "cancel":
        # dims d % 4 != 1: +-3 x the same large key value in the two halves (they cancel exactly);
        # dims d % 4 == 1: small products, added while the partial sum is large
        big = rng.choice(grid[np.abs(grid) >= 64], size=(N, D // 2)).astype(np.float32)
        k = np.concatenate([big, big], axis=1)
        q = np.concatenate([np.full((H, D // 2), 3.0), np.full((H, D // 2), -3.0)], axis=1).astype(np.float32)
        small = np.arange(D) % 4 == 1
        q[:, small] = _bf16(rng.standard_normal((H, int(small.sum()))) * 2.0 ** -12)
        k[:, small] = rng.choice(grid[np.abs(grid) <= 4], size=(N, int(small.sum())))
    elif case == "subnormal":
        q = _bf16(rng.standard_normal((H, D)) * 2.0 ** -124)
        ks = np.ones(N, dtype=np.float32)
    elif case == "wide_scale":
        ks = (2.0 ** rng.integers(-60, 60, N)).astype(np.float32)
    return q, k, ks, w


@pytest.mark.parametrize("case", ["gauss", "cancel", "subnormal", "wide_scale"])
@pytest.mark.parametrize("model", MODELS, ids=lambda m: m.__name__[7:])
def test_cert_bound_holds(case, model):
    rng = np.random.default_rng(["gauss", "cancel", "subnormal", "wide_scale"].index(case))
    q, k, ks, w = _inputs(case, rng)
    s = oidx.indexer_score(q[None], k, ks, w[None])[0].astype(np.float64)
    a, dots, P = model(q, k, w, ks)
    err = np.abs(s - a.astype(np.float64))
    e = _bound(a.astype(np.float64), ks.astype(np.float64), w, dots, P)
    assert np.all(np.isfinite(e))
    worst = float(np.max(err / e))
    assert worst <= 1 / 3, f"bound used up to {worst:.3f} of its width"
    # the adversarial cases need the term they were built for
    if case == "cancel":
        e_no = _bound(a.astype(np.float64), ks.astype(np.float64), w, dots, P, use_pw=False)
        assert np.any(err > e_no), "cancellation case does not stress the PW term"
    if case == "subnormal" and model is _model_ftz:
        e_no = _bound(a.astype(np.float64), ks.astype(np.float64), w, dots, P, use_tiny=False)
        assert np.any(err > e_no), "subnormal case does not stress the absolute term"
