"""Pins of the DG-Indexer oracle (oracle/indexer.py) by known answers from the
reference's own tests, closed forms and library routines -- never by restating
the oracle's formula.

Known answers: needle and padding centroids (test_triton_indexer.py:147-168),
zeros in / zeros out (:488-497), the ``-0.75 ln 3`` score (test_indexer.py:143-164),
the causal ``-inf`` pattern (test_indexer.py:169-206), the penalty order
``[3, 2, 1, 0]`` (test_triton_indexer.py:247-255) and the budget clamp (:257-265).
"""
import math

import numpy as np

from oracle import indexer as oidx


def test_centroid_needle_in_haystack():
    k = np.full((1, 256, 64), 0.01)
    k[0, 70, :] = 10.0
    c = oidx.compute_centroids(k, 64)
    pure_mean = (63 * 0.01 + 10.0) / 64.0
    assert c[0, 1, 0] > 30 * pure_mean
    assert abs(c[0, 1, 0] - 0.5 * (pure_mean + 10.0)) < 1e-12
    assert np.allclose(c[0, 0], 0.01) and np.allclose(c[0, 2:], 0.01)


def test_centroid_zero_padding_counts():
    c = oidx.compute_centroids(np.full((1, 100, 64), -2.0), 64)
    assert c.shape == (1, 2, 64)
    assert np.allclose(c[0, 0], -2.0)
    # 36 tokens of -2 and 28 zeros of padding: mean -72/64, max 0
    assert np.allclose(c[0, 1], 0.5 * (-72.0 / 64.0 + 0.0))


def test_centroid_zeros_and_empty():
    assert (oidx.compute_centroids(np.zeros((2, 128, 64)), 64) == 0).all()
    assert oidx.compute_centroids(np.zeros((2, 0, 8)), 64).shape == (2, 0, 8)


def test_centroid_brute_force_small():
    """Per-block loops over explicit token lists on a ragged tail (bs = 16, L = 37)."""
    r = np.random.default_rng(0)
    k = r.standard_normal((2, 37, 3))
    c = oidx.compute_centroids(k, 16)
    for b in range(2):
        for n in range(3):
            toks = [k[b, t] for t in range(16 * n, min(16 * n + 16, 37))]
            toks += [np.zeros(3)] * (16 - len(toks))
            mean = sum(toks) / 16.0
            mx = np.array([max(t[j] for t in toks) for j in range(3)])
            assert np.allclose(c[b, n], 0.5 * (mean + mx))


def test_prefill_log_distance_known_answer():
    s = oidx.prefill_scores(np.zeros((1, 256, 32)), np.zeros((1, 4, 32)), 0.75, 64)
    assert math.isclose(s[0, 192, 1], -0.75 * math.log(3.0), rel_tol=1e-12)


def test_prefill_causal_pattern():
    r = np.random.default_rng(1)
    s = oidx.prefill_scores(r.standard_normal((1, 512, 32)), r.standard_normal((1, 8, 32)), 0.5, 64)
    for t in [0, 31, 63, 64, 127, 250, 511]:
        qb = t // 64
        assert np.isneginf(s[0, t, qb + 1:]).all()
        assert np.isfinite(s[0, t, : qb + 1]).all()


def test_prefill_penalty_order():
    d = 64
    s = oidx.prefill_scores(np.ones((1, 256, d)) / math.sqrt(d), np.ones((1, 4, d)) / math.sqrt(d), 1.0, 64)
    assert oidx.topk_desc(s[0, 255], 4).tolist() == [3, 2, 1, 0]


def test_budget_clamp_single_block():
    r = np.random.default_rng(2)
    s = oidx.prefill_scores(r.standard_normal((2, 32, 64)), r.standard_normal((2, 1, 64)), 0.5, 64)
    idx = oidx.topk_desc(s, 32)
    assert idx.shape == (2, 32, 1) and (idx == 0).all()


def test_dot_term_is_scaled_inner_product():
    """Zero penalty: the score is q.c / sqrt(d), checked on orthonormal directions."""
    d = 16
    q = np.zeros((1, 1, d)); q[0, 0, 3] = 2.0
    c = np.zeros((1, 4, d)); c[0, 1, 3] = 5.0; c[0, 2, 4] = 7.0
    s = oidx.decode_scores(q, c, 0.0)
    assert np.allclose(s[0, 0], [0.0, 10.0 / 4.0, 0.0, 0.0])


def test_decode_penalty_closed_form():
    nb = 10
    s = oidx.decode_scores(np.zeros((1, 1, 8)), np.zeros((1, nb, 8)), 0.3)
    assert s[0, 0, nb - 1] == 0.0
    assert math.isclose(s[0, 0, 0], -0.3 * math.log(10.0), rel_tol=1e-12)
    assert (np.diff(s[0, 0]) > 0).all()          # newer blocks are penalised less


def test_decode_equals_prefill_row_in_last_block():
    """The decode query at position L-1 scores like the prefill row of that token
    (same last block, every block causal-visible)."""
    r = np.random.default_rng(3)
    L, d, nb = 300, 32, 5
    q = r.standard_normal((1, L, d))
    c = r.standard_normal((1, nb, d))
    pre = oidx.prefill_scores(q, c, 0.4, 64)[0, L - 1]
    dec = oidx.decode_scores(q[:, L - 1:L], c, 0.4)[0, 0]
    assert np.allclose(pre, dec)


def test_topk_desc_matches_stable_argsort():
    """Score descending, ties by lower index: numpy's stable argsort of -score."""
    r = np.random.default_rng(4)
    s = r.integers(0, 5, size=(50, 40)).astype(np.float64)     # heavy ties
    got = oidx.topk_desc(s, 12)
    exp = np.argsort(-s, axis=-1, kind="stable")[:, :12]
    assert (got == exp).all()


def test_decode_tail_centroid():
    """A cache of 70 keys: one complete block and a 6-token tail padded with 58 zeros."""
    k = np.zeros((1, 70, 2))
    k[0, :64] = 1.0
    k[0, 64:, 0] = 3.0
    k[0, 64:, 1] = -1.0
    c = oidx.decode_centroid_cache(k, 64)
    assert c.shape == (1, 2, 2)
    assert np.allclose(c[0, 0], 1.0)
    assert np.allclose(c[0, 1], [0.5 * (18.0 / 64 + 3.0), 0.5 * (-6.0 / 64 + 0.0)])


def test_top_gap():
    assert oidx.top_gap([5.0, 1.0, 3.0, 2.0], 2) == 1.0
    assert oidx.top_gap([1.0, 2.0], 2) == np.inf


def test_prefill_scores_at_chosen_positions():
    """Rows scored at given positions equal those rows of the full causal matrix, including
    a row in the first block (one live centroid) and rows on block edges."""
    rng = np.random.default_rng(11)
    q = rng.standard_normal((2, 300, 16))
    c = rng.standard_normal((2, 5, 16))
    full = oidx.prefill_scores(q, c, 0.3, block_size=64)
    rows = np.array([0, 63, 64, 130, 255, 256, 299])
    part = oidx.prefill_scores(q[:, rows], c, 0.3, block_size=64, positions=rows)
    assert np.array_equal(np.isinf(part), np.isinf(full[:, rows]))
    fin = np.isfinite(part)
    assert np.allclose(part[fin], full[:, rows][fin], rtol=0, atol=1e-12)
