"""Pins oracle.indexer: the C score chain against exact rational arithmetic, the C top-k against a
Python sort with the same tie rule, and the take-all case against the reference's index build."""
import numpy as np

from oracle import indexer as oi
from oracle import sparse_attn as osa


def test_score_chain_bit_exact_vs_rational_bruteforce():
    rng = np.random.default_rng(0)
    S, H, D, N = 2, 3, 5, 7
    q = rng.standard_normal((S, H, D)).astype(np.float32)
    k = rng.standard_normal((N, D)).astype(np.float32)
    w = rng.standard_normal((S, H)).astype(np.float32)
    ks = np.abs(rng.standard_normal(N)).astype(np.float32) + 0.5
    nvis = np.array([7, 4], dtype=np.int32)
    got = oi.indexer_score(q, k, ks, w, nvis)
    ref = oi.score_bruteforce(q, k, ks, w, nvis)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.all(np.isneginf(got[1, 4:]))


def test_score_relu_and_zero_handling():
    # every dot product negative -> all ReLUs 0 -> score +0 regardless of weights
    q = -np.ones((1, 2, 4), np.float32)
    k = np.ones((3, 4), np.float32)
    w = np.array([[-1.0, 2.0]], np.float32)
    s = oi.indexer_score(q, k, None, w)
    assert np.all(s == 0) and not np.any(np.signbit(s))


def test_topk_tie_rule_and_order():
    s = np.array([[1.0, 3.0, 3.0, -0.0, 0.0, 3.0, 2.0, 0.0]], np.float32)
    # ranking: 3.0 at 1,2,5 ; 2.0 at 6 ; 1.0 at 0 ; zeros (-0 == +0) at 3,4,7
    assert oi.topk(s, 2).tolist() == [[1, 2]]
    assert oi.topk(s, 4).tolist() == [[1, 2, 5, 6]]
    assert oi.topk(s, 6).tolist() == [[0, 1, 2, 3, 5, 6]]          # -0 at 3 ties +0, lowest index wins
    assert oi.topk(s, 10).tolist() == [[0, 1, 2, 3, 4, 5, 6, 7, -1, -1]]
    assert oi.topk(s, 3, nvis=np.array([2], np.int32)).tolist() == [[0, 1, -1]]


def test_topk_matches_python_sort():
    rng = np.random.default_rng(5)
    s = rng.integers(-5, 6, (20, 300)).astype(np.float32) * 0.5      # many exact ties
    nvis = rng.integers(0, 301, 20).astype(np.int32)
    for k in (1, 17, 150, 300, 400):
        np.testing.assert_array_equal(oi.topk(s, k, nvis), oi.topk_bruteforce(s, k, nvis))


def test_take_all_equals_reference_index_build():
    # nvis <= k: the selection is every causally visible compressed row, as in the engine
    rng = np.random.default_rng(6)
    pos, ratio, n_comp, k = 1000, 4, 400, 2048
    nvis = (pos + 1) // ratio
    s = rng.standard_normal((1, n_comp)).astype(np.float32)
    sel = oi.topk(s, k, np.array([min(nvis, n_comp)], np.int32))[0]
    eng = osa.engine_decode_idxs(pos, 128, n_comp, ratio).numpy()[128:] - 128
    np.testing.assert_array_equal(sel[: len(eng)], eng)
    assert np.all(sel[len(eng):] == -1)
