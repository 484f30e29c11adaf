"""MABA-SA decode oracle -- TEST INFRASTRUCTURE ONLY.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg.  Never imported by the product package.

All streams are softmax attention over an explicit key set, computed in
float64 with the reference's per-head up-projected keys and values
(``k_h = W_k[h] c``, ``v_h = W_v[h] c``; layers/sparse_attention.py:253-254),
i.e. without the latent absorption the HIP kernel uses, so that the
absorption identity is checked too.

Functions
---------
``local_keys``          key positions of the local stream at decode:
                        sinks ``[0, min(4,L))`` plus ``[max(min(4,L), L-128), L)``
                        (sparse_attention.py:84-93; for ``L <= 132`` the
                        masked branch :95-105 selects the same set).
``local_stream``        softmax over ``local_keys``.
``sparse_stream``       softmax over the tokens of the selected 64-blocks with
                        position ``< L`` (sparse_attention.py:129-143).  Index
                        sets ``[B, 1, K]`` are shared by all heads (reference
                        semantics, :130-131); ``[B, H, K]`` gives one set per
                        head.
``hca_stream``          compressed-prefix stream at position ``pos = L-1``
                        (sparse_attention.py:173-219): ``pos < 63`` returns
                        ``W_v`` applied to the running mean of ``c[0..pos]``
                        (:189-199); otherwise softmax over the means of all
                        complete 64-blocks up-projected by ``W_k``/``W_v``
                        (:201-217).  ``means`` may be passed in (for a cache
                        stored in bf16) instead of being recomputed.
``superposition``       ``g0*o_local + g1*o_sparse + g2*o_hca`` with
                        ``g = softmax(logits)`` or given weights; 3-D gates
                        broadcast over heads, 4-D gates are per head
                        (common.py:406-438, cpu_indexer.py:115-150).
``maba_sa_decode``      the composition of the three streams and the gate
                        (sparse_attention.py:263-275), before ``o_proj``.

``maba_sa_prefill_heads``  every query of a prefill (sparse_attention.py:95-105,
                        145-171, 173-219, 275) from per-head keys and values, as
                        explicit dense masks over [Lq, Lkv]: the local window and
                        sinks, each query's selected blocks with multiplicity and
                        ``token <= pos``, the complete means with
                        ``(e+1) pool - 1 <= pos`` (or the given running-mean row
                        before ``pool - 1``), then the gate.
``maba_sa_prefill``     the same from the latent cache and ``W_k``/``W_v``.  Pinned
                        against ``maba_sa_decode`` run at every prefix length
                        ``L = pos + 1`` (a decode step is the last prefill row).

Pinned by: partition of unity and extreme logits (test_triton_indexer.py:
326-346), a single-key stream returning that key's value, uniform scores
returning the mean value, brute-force dense masked softmax on tiny shapes and
the float64 absorption identity ``<q, W_k c> = <W_k^T q, c>``.
"""
from __future__ import annotations

import math

import numpy as np


def _softmax_attend(q, keys, vals, scale):
    """``softmax(q.keys^T * scale) vals`` for q ``[dh]``, keys/vals ``[n, dh]``."""
    if keys.shape[0] == 0:
        return np.zeros(vals.shape[-1])
    s = keys @ q * scale
    m = s.max()
    p = np.exp(s - m)
    return (p / p.sum()) @ vals


def _heads(W, H):
    """Split an ``nn.Linear(d_c, H*dh)`` weight ``[H*dh, d_c]`` into ``[H, dh, d_c]``."""
    W = np.asarray(W, np.float64)
    return W.reshape(H, W.shape[0] // H, W.shape[1])


def local_keys(L, window=128, n_sink=4):
    """Positions attended by the local stream of a decode step with L keys."""
    ns = min(n_sink, L)
    start = max(ns, L - window)
    return np.concatenate([np.arange(ns), np.arange(start, L)]).astype(np.int64)


def local_stream(q, c_kv, Wk, Wv, L=None, window=128, n_sink=4):
    """Local stream output ``[B, H, dh]`` (sparse_attention.py:84-93)."""
    q = np.asarray(q, np.float64)
    B, H, dh = q.shape
    c = np.asarray(c_kv, np.float64)
    L = c.shape[1] if L is None else L
    Wk_h, Wv_h = _heads(Wk, H), _heads(Wv, H)
    pos = local_keys(L, window, n_sink)
    out = np.zeros((B, H, dh))
    scale = 1.0 / math.sqrt(dh)
    for b in range(B):
        cs = c[b, pos]                                  # [n, d_c]
        for h in range(H):
            out[b, h] = _softmax_attend(q[b, h], cs @ Wk_h[h].T, cs @ Wv_h[h].T, scale)
    return out


def sparse_positions(idx_row, L, block_size=64):
    """Token positions of the selected blocks that are ``< L`` (sparse_attention.py:136-141)."""
    idx_row = np.asarray(idx_row, np.int64)
    pos = (idx_row[:, None] * block_size + np.arange(block_size)[None, :]).reshape(-1)
    return pos[pos < L]


def sparse_stream(q, c_kv, Wk, Wv, idx, L=None, block_size=64):
    """Sparse stream output ``[B, H, dh]`` (sparse_attention.py:129-143)."""
    q = np.asarray(q, np.float64)
    B, H, dh = q.shape
    c = np.asarray(c_kv, np.float64)
    L = c.shape[1] if L is None else L
    idx = np.asarray(idx, np.int64)
    Wk_h, Wv_h = _heads(Wk, H), _heads(Wv, H)
    out = np.zeros((B, H, dh))
    scale = 1.0 / math.sqrt(dh)
    for b in range(B):
        for h in range(H):
            row = idx[b, 0] if idx.shape[1] == 1 else idx[b, h]
            pos = sparse_positions(row, L, block_size)
            cs = c[b, pos]
            out[b, h] = _softmax_attend(q[b, h], cs @ Wk_h[h].T, cs @ Wv_h[h].T, scale)
    return out


def hca_means(c_kv, L=None, pool=64):
    """Means of the complete ``pool``-token blocks of the latent cache (sparse_attention.py:206)."""
    c = np.asarray(c_kv, np.float64)
    L = c.shape[1] if L is None else L
    nc = L // pool
    return c[:, : nc * pool].reshape(c.shape[0], nc, pool, c.shape[2]).mean(axis=2)


def hca_stream(q, c_kv, Wk, Wv, L=None, pool=64, means=None):
    """HCA stream output ``[B, H, dh]`` for the query at position ``L-1``."""
    q = np.asarray(q, np.float64)
    B, H, dh = q.shape
    c = np.asarray(c_kv, np.float64)
    L = c.shape[1] if L is None else L
    Wk_h, Wv_h = _heads(Wk, H), _heads(Wv, H)
    out = np.zeros((B, H, dh))
    pos = L - 1
    scale = 1.0 / math.sqrt(dh)
    if pos < pool - 1:                                   # sparse_attention.py:186-199
        cm = c[:, : pos + 1].mean(axis=1)               # running mean of c[0..pos]
        for h in range(H):
            out[:, h] = cm @ Wv_h[h].T
        return out
    cbar = hca_means(c, L, pool) if means is None else np.asarray(means, np.float64)[:, : L // pool]
    for b in range(B):
        for h in range(H):
            out[b, h] = _softmax_attend(q[b, h], cbar[b] @ Wk_h[h].T, cbar[b] @ Wv_h[h].T, scale)
    return out


def superposition(o_local, o_sparse, o_hca, gate_logits=None, gate_weights=None):
    """Gate superposition (common.py:406-438); 3-D gates ``[B,L,3]``, 4-D ``[B,H,L,3]``."""
    ol, os_, oh = (np.asarray(x, np.float64) for x in (o_local, o_sparse, o_hca))
    if gate_weights is not None:
        g = np.asarray(gate_weights, np.float64)
    else:
        z = np.asarray(gate_logits, np.float64)
        z = z - z.max(axis=-1, keepdims=True)
        g = np.exp(z) / np.exp(z).sum(axis=-1, keepdims=True)
    if g.ndim == 3:
        g = g[:, None]                                   # broadcast over heads
    return g[..., 0:1] * ol + g[..., 1:2] * os_ + g[..., 2:3] * oh


def maba_sa_decode(q, c_kv, Wk, Wv, idx, gate_logits, L=None, window=128,
                   n_sink=4, block_size=64, pool=64, means=None):
    """Fused MABA-SA decode ``[B, H, dh]`` before ``o_proj`` (sparse_attention.py:263-275).

    ``gate_logits`` is ``[B, 3]`` (one decode token) or ``[B, H, 3]``.
    """
    ol = local_stream(q, c_kv, Wk, Wv, L, window, n_sink)
    os_ = sparse_stream(q, c_kv, Wk, Wv, idx, L, block_size)
    oh = hca_stream(q, c_kv, Wk, Wv, L, pool, means)
    g = np.asarray(gate_logits, np.float64)
    g4 = g[:, None, None, :] if g.ndim == 2 else g[:, :, None, :]
    out = superposition(ol[:, :, None], os_[:, :, None], oh[:, :, None], gate_logits=g4)
    return out[:, :, 0]


def maba_sa_prefill_heads(q, k, v, kh, vh, early, idx, gate_logits, window=128, n_sink=4,
                          block_size=64, pool=64, scale=None):
    """Prefill output ``[B, H, Lq, dh]`` from per-head q ``[B,H,Lq,dh]``, k/v ``[B,H,Lkv,dh]``,
    kh/vh ``[B,H,Lkv//pool,dh]``, early ``[B,H,n_early,dh]`` (rows for pos < pool-1) or
    None, idx ``[B,Lq|1,K]`` and gate logits ``[B,Lq,3]`` or ``[B,H,Lq,3]``."""
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    B, H, Lq, dh = q.shape
    Lkv = k.shape[2]
    scale = 1.0 / math.sqrt(dh) if scale is None else scale
    pos = (Lkv - Lq) + np.arange(Lq)
    j = np.arange(Lkv)
    ns = min(n_sink, Lkv)
    idx = np.asarray(idx, np.int64)
    nc = Lkv // pool

    def attend(s, w, vals):      # rows of scores s with multiplicities w (0 = masked)
        s = np.where(w > 0, s, -np.inf)
        m = s.max(axis=-1, keepdims=True)
        m = np.where(np.isfinite(m), m, 0.0)
        p = w * np.exp(s - m)
        tot = p.sum(axis=-1, keepdims=True)
        return np.where(tot > 0, (p / np.where(tot > 0, tot, 1.0)) @ vals, 0.0)

    local_w = ((j[None] <= pos[:, None]) &
               (((pos[:, None] - j[None]) < window) | (j[None] < ns))).astype(np.float64)
    nb = (Lkv + block_size - 1) // block_size
    out = np.zeros((B, H, Lq, dh))
    for b in range(B):
        sp_w = np.zeros((Lq, Lkv))
        for t in range(Lq):
            row = idx[b, t] if idx.shape[1] == Lq else idx[b, 0]
            for blk in row:
                if 0 <= blk < nb:
                    toks = np.arange(blk * block_size, min((blk + 1) * block_size, Lkv))
                    toks = toks[toks <= pos[t]]
                    sp_w[t, toks] += 1.0
        hca_w = (((np.arange(nc) + 1) * pool - 1)[None] <= pos[:, None]).astype(np.float64)
        for h in range(H):
            s = q[b, h] @ k[b, h].T * scale
            ol = attend(s, local_w, v[b, h])
            os_ = attend(s, sp_w, v[b, h])
            if nc > 0:
                khb, vhb = np.asarray(kh, np.float64)[b, h], np.asarray(vh, np.float64)[b, h]
                oh = attend(q[b, h] @ khb.T * scale, hca_w, vhb)
            else:
                oh = np.zeros((Lq, dh))
            for t in range(Lq):
                if pos[t] < pool - 1:
                    oh[t] = np.asarray(early, np.float64)[b, h, t]
            g = np.asarray(gate_logits, np.float64)
            g = g[b] if g.ndim == 3 else g[b, h]
            g = np.exp(g - g.max(axis=-1, keepdims=True))
            g = g / g.sum(axis=-1, keepdims=True)
            out[b, h] = g[:, 0:1] * ol + g[:, 1:2] * os_ + g[:, 2:3] * oh
    return out


def maba_sa_prefill(q, c_kv, Wk, Wv, idx, gate_logits, Lq=None, window=128, n_sink=4,
                    block_size=64, pool=64):
    """Prefill from the latent cache ``c_kv [B, Lkv, d_c]``: the last ``Lq`` positions are the
    queries (``q [B, H, Lq, dh]``); keys, values and the complete-block means are up-projected
    per head, and the rows before ``pool - 1`` take ``W_v`` of the running mean."""
    q = np.asarray(q, np.float64)
    B, H, Lq_, dh = q.shape
    c = np.asarray(c_kv, np.float64)
    Lkv = c.shape[1]
    Wk_h, Wv_h = _heads(Wk, H), _heads(Wv, H)
    k = np.einsum("bld,hed->bhle", c, Wk_h)
    v = np.einsum("bld,hed->bhle", c, Wv_h)
    means = hca_means(c, Lkv, pool)
    kh = np.einsum("bnd,hed->bhne", means, Wk_h)
    vh = np.einsum("bnd,hed->bhne", means, Wv_h)
    off = Lkv - Lq_
    n_early = max(0, min(Lq_, pool - 1 - off))
    early = np.zeros((B, H, max(n_early, 1), dh))
    for t in range(n_early):
        cm = c[:, : off + t + 1].mean(axis=1)
        early[:, :, t] = np.einsum("bd,hed->bhe", cm, Wv_h)
    return maba_sa_prefill_heads(q, k, v, kh, vh, early, idx, gate_logits, window, n_sink, block_size, pool)
