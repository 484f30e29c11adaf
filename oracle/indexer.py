"""DG-Indexer oracle -- TEST INFRASTRUCTURE ONLY.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg.  Never imported by the product package.

Functions
---------
``compute_centroids``  ``c_n = 0.5*(mean + max)`` over 64-token blocks; the
                       last block is zero-padded and the zeros take part in
                       both the mean (divide by block size) and the max
                       (common.py:343-350, cpu_indexer.py:38-50).  Output
                       is rounded to the input dtype by the caller
                       (cpu_indexer.py:50).  Pinned by the needle and padding
                       known answers (test_triton_indexer.py:147-168) and
                       zeros-in/zeros-out (test_triton_indexer.py:488-497).
``prefill_scores``     causal prefill scores ``(q_t/sqrt d).c_n -
                       lam*log1p(|t//bs - n|)``, ``-inf`` for ``n > t//bs``
                       (cpu_indexer.py:91-102), in float64.  Pinned by the
                       ``-0.75*ln 3`` known answer (test_indexer.py:143-164),
                       the causal pattern (test_triton_indexer.py:222-244) and
                       the penalty order ``[3,2,1,0]``
                       (test_triton_indexer.py:247-255).  Chosen rows
                       (``positions``) equal the same rows of the full matrix.
``decode_scores``      decode scores with ``q_blk = nb-1`` and no mask
                       (layers/indexer.py:101-107).  Pinned by the same
                       penalty closed form and brute force on tiny inputs.
``topk_desc``          selection of the top ``min(K, nb)`` entries sorted by
                       score descending, ties by index ascending.  torch.topk
                       leaves tie order unspecified (cpu_indexer.py:107-108), so
                       tied orders are "parity unpinned" and the tests compare
                       selections only where the score gap exceeds 1e-4.
``decode_centroid_cache`` the per-step centroid cache of
                       layers/indexer.py:62-81: complete blocks plus the
                       zero-padded partial tail block.
"""
from __future__ import annotations

import math

import numpy as np


def compute_centroids(k_idx, block_size=64):
    """Block centroids ``0.5*(mean+max)`` in float64 (common.py:329-350)."""
    k = np.asarray(k_idx, np.float64)
    B, L, d = k.shape
    if L == 0:
        return np.zeros((B, 0, d))
    nb = (L + block_size - 1) // block_size
    pad = nb * block_size - L
    kp = np.concatenate([k, np.zeros((B, pad, d))], axis=1) if pad else k
    kb = kp.reshape(B, nb, block_size, d)
    return 0.5 * (kb.mean(axis=2) + kb.max(axis=2))


def prefill_scores(q_idx, centroids, lam, block_size=64, positions=None):
    """Causal prefill score matrix ``[B, L, nb]`` (cpu_indexer.py:91-102).

    ``positions`` (default ``0 .. L-1``) are the token positions of the query rows, so that
    chosen rows of a long prefill can be scored without the whole matrix."""
    q = np.asarray(q_idx, np.float64)
    c = np.asarray(centroids, np.float64)
    B, L, d = q.shape
    nb = c.shape[1]
    scale = 1.0 / math.sqrt(d)
    s = np.einsum("bld,bnd->bln", q * scale, c)
    pos = np.arange(L) if positions is None else np.asarray(positions, np.int64)
    qi = (pos // block_size)[:, None]
    ni = np.arange(nb)[None, :]
    pen = lam * np.log1p(np.abs(qi - ni).astype(np.float64))
    sc = s - pen[None]
    sc = np.where((ni > qi)[None], -np.inf, sc)
    return sc


def decode_scores(q, centroids, lam):
    """Decode scores ``[B, Hq, nb]`` for queries ``q [B, Hq, d]``.

    ``q_blk = nb - 1``; ``dist = max(q_blk - n, 0)``; no causal mask
    (layers/indexer.py:101-107).  ``Hq`` generalises the reference's single
    indexer query to several query heads sharing one centroid set.
    """
    q = np.asarray(q, np.float64)
    c = np.asarray(centroids, np.float64)
    d = q.shape[-1]
    nb = c.shape[1]
    scale = 1.0 / math.sqrt(d)
    dot = np.einsum("bhd,bnd->bhn", q * scale, c)
    dist = np.maximum((nb - 1) - np.arange(nb), 0).astype(np.float64)
    return dot - (lam * np.log1p(dist))[None, None, :]


def topk_desc(scores, k):
    """Indices of the top ``min(k, n)`` scores along the last axis.

    Sorted by score descending, ties broken by the lower index first.
    """
    s = np.asarray(scores, np.float64)
    n = s.shape[-1]
    ak = min(k, n)
    idx = np.arange(n)
    flat = s.reshape(-1, n)
    out = np.empty((flat.shape[0], ak), np.int64)
    for r in range(flat.shape[0]):
        order = np.lexsort((idx, -flat[r]))   # primary: -score, secondary: index
        out[r] = order[:ak]
    return out.reshape(s.shape[:-1] + (ak,))


def decode_centroid_cache(k_idx_cache, block_size=64):
    """Centroids seen by a decode step whose key cache is ``k_idx_cache [B, L, d]``.

    Complete blocks each give one centroid; a partial tail block gives the
    zero-padded tail centroid (layers/indexer.py:62-81).  The result equals
    ``compute_centroids`` over the whole cache because a block's centroid only
    depends on its own tokens.
    """
    return compute_centroids(k_idx_cache, block_size)


def top_gap(scores_row, k):
    """Gap between the k-th and (k+1)-th best score of one row (inf if n <= k)."""
    s = np.sort(np.asarray(scores_row, np.float64))[::-1]
    if s.shape[0] <= k:
        return np.inf
    return s[k - 1] - s[k]
