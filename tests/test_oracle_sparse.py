"""Pins of the MABA-SA decode oracle (oracle/sparse_attn.py).

Each stream is softmax attention over an explicit key set; the tests fix the
key sets by hand (sparse_attention.py:84-93, :129-143, :173-219), check
single-key and uniform-score closed forms, the gate's partition of unity and
extreme logits (test_triton_indexer.py:326-346), a dense masked softmax on a
short cache (the reference's masked branch, sparse_attention.py:95-105), and the
latent-absorption identity the HIP kernel relies on.
"""
import math

import numpy as np
import pytest

from oracle import sparse_attn as osa


def _case(B=2, H=3, dh=8, dc=16, L=300, seed=0):
    r = np.random.default_rng(seed)
    c = r.standard_normal((B, L, dc))
    Wk = r.standard_normal((H * dh, dc)) * 0.3
    Wv = r.standard_normal((H * dh, dc)) * 0.3
    q = r.standard_normal((B, H, dh))
    return q, c, Wk, Wv


def test_local_keys_known_sets():
    assert osa.local_keys(1).tolist() == [0]
    assert osa.local_keys(4).tolist() == [0, 1, 2, 3]
    assert osa.local_keys(10).tolist() == list(range(10))
    assert osa.local_keys(132).tolist() == list(range(132))
    assert osa.local_keys(133).tolist() == [0, 1, 2, 3] + list(range(5, 133))
    k = osa.local_keys(1_000_000)
    assert k.shape == (132,) and k[4] == 1_000_000 - 128 and k[-1] == 999_999


def test_sparse_positions_mask_beyond_L():
    pos = osa.sparse_positions([0, 2, 5], L=150, block_size=64)
    assert pos.tolist() == list(range(64)) + list(range(128, 150))


def test_single_key_returns_its_value():
    q, c, Wk, Wv = _case(L=64)
    out = osa.sparse_stream(q, c, Wk, Wv, np.zeros((2, 1, 1), np.int64), L=1)
    for b in range(2):
        for h in range(3):
            assert np.allclose(out[b, h], Wv.reshape(3, 8, 16)[h] @ c[b, 0])


def test_uniform_scores_give_mean_value():
    q, c, Wk, Wv = _case(L=200)
    out = osa.local_stream(np.zeros_like(q), c, Wk, Wv)
    keys = osa.local_keys(200)
    for h in range(3):
        exp = Wv.reshape(3, 8, 16)[h] @ c[:, keys].mean(axis=1).T
        assert np.allclose(out[:, h], exp.T)


def test_local_stream_short_cache_is_dense_softmax():
    """L <= 132: the local key set is the whole cache, so the stream is plain softmax
    attention over all keys (the reference's masked dense branch at the last row)."""
    q, c, Wk, Wv = _case(L=50, seed=1)
    out = osa.local_stream(q, c, Wk, Wv)
    Wk_h, Wv_h = Wk.reshape(3, 8, 16), Wv.reshape(3, 8, 16)
    for b in range(2):
        for h in range(3):
            K = c[b] @ Wk_h[h].T
            V = c[b] @ Wv_h[h].T
            z = K @ q[b, h] / math.sqrt(8)
            p = np.exp(z - z.max()); p /= p.sum()
            assert np.allclose(out[b, h], p @ V)


def test_hca_early_running_mean():
    q, c, Wk, Wv = _case(L=10, seed=2)
    out = osa.hca_stream(q, c, Wk, Wv)
    for h in range(3):
        assert np.allclose(out[:, h], (Wv.reshape(3, 8, 16)[h] @ c.mean(axis=1).T).T)


def test_hca_means_known_answer():
    c = np.arange(2 * 130 * 1, dtype=np.float64).reshape(2, 130, 1)
    m = osa.hca_means(c, pool=64)
    assert m.shape == (2, 2, 1)                   # the partial third block is excluded
    assert np.allclose(m[0, :, 0], [31.5, 95.5]) and np.allclose(m[1, :, 0], [161.5, 225.5])


def test_superposition_partition_of_unity_and_extremes():
    r = np.random.default_rng(3)
    x = r.standard_normal((2, 4, 64, 16))
    assert np.allclose(osa.superposition(x, x, x, gate_logits=r.standard_normal((2, 64, 3))), x)
    ol, os_, oh = (np.full((1, 2, 4, 8), v) for v in (1.0, 2.0, 3.0))
    out = osa.superposition(ol, os_, oh, gate_logits=np.array([[[1e4, -1e4, -1e4]] * 4]))
    assert np.isfinite(out).all() and np.allclose(out, ol)
    w = np.array([[[0.2, 0.3, 0.5]]])
    assert np.allclose(osa.superposition(ol[:, :, :1], os_[:, :, :1], oh[:, :, :1], gate_weights=w), 2.3)


def test_latent_absorption_identity():
    """<q_h, W_k,h c> = <W_k,h^T q_h, c> and sum_j p_j W_v,h c_j = W_v,h sum_j p_j c_j:
    the fused decode computed entirely in latent space equals the oracle's
    explicit up-projection, in float64."""
    B, H, dh, dc, L = 2, 3, 8, 16, 700
    q, c, Wk, Wv = _case(B, H, dh, dc, L, seed=4)
    r = np.random.default_rng(5)
    idx = np.stack([np.stack([r.permutation(11)[:4] for _ in range(H)]) for _ in range(B)])
    gate = r.standard_normal((B, 3))
    exp = osa.maba_sa_decode(q, c, Wk, Wv, idx, gate)
    Wk_h, Wv_h = Wk.reshape(H, dh, dc), Wv.reshape(H, dh, dc)
    q_lat = np.einsum("bhd,hdc->bhc", q, Wk_h)
    scale = 1 / math.sqrt(dh)
    means = c[:, : (L // 64) * 64].reshape(B, L // 64, 64, dc).mean(axis=2)
    g = np.exp(gate - gate.max(-1, keepdims=True)); g /= g.sum(-1, keepdims=True)
    got = np.zeros((B, H, dh))
    for b in range(B):
        for h in range(H):
            sets = [c[b, osa.local_keys(L)],
                    c[b, osa.sparse_positions(idx[b, h], L)],
                    means[b]]
            z = np.zeros(dc)
            for s, rows in enumerate(sets):
                e = rows @ q_lat[b, h] * scale
                p = np.exp(e - e.max()); p /= p.sum()
                z += g[b, s] * (p @ rows)
            got[b, h] = Wv_h[h] @ z
    assert np.allclose(got, exp, rtol=1e-12, atol=1e-12)


# ----------------------------------------------------------------------------- prefill streams

@pytest.mark.parametrize("Lkv,Lq,window,n_sink,K", [(150, 150, 128, 4, 3), (300, 77, 40, 2, 4),
                                                    (70, 70, 16, 0, 2), (500, 33, 128, 4, 5)])
def test_prefill_rows_equal_decode_at_each_prefix(Lkv, Lq, window, n_sink, K):
    """A decode step is the last row of a prefill: every prefill row equals the decode oracle
    run on the prefix that ends at its position, with that row's blocks and gate."""
    rng = np.random.default_rng(Lkv + Lq)
    B, H, dh, dc = 2, 3, 8, 12
    c = rng.standard_normal((B, Lkv, dc))
    Wk = rng.standard_normal((H * dh, dc)) * 0.3
    Wv = rng.standard_normal((H * dh, dc))
    q = rng.standard_normal((B, H, Lq, dh))
    nb = (Lkv + 63) // 64
    idx = rng.integers(0, nb, size=(B, Lq, K))
    idx[0, 0, 1] = idx[0, 0, 0]                     # a repeated block counts twice
    gate = rng.standard_normal((B, Lq, 3))
    got = osa.maba_sa_prefill(q, c, Wk, Wv, idx, gate, window=window, n_sink=n_sink)
    off = Lkv - Lq
    for t in range(Lq):
        L = off + t + 1
        exp = osa.maba_sa_decode(q[:, :, t], c[:, :L], Wk, Wv, idx[:, t:t + 1], gate[:, t], window=window,
                                 n_sink=n_sink)
        assert np.allclose(got[:, :, t], exp, rtol=1e-10, atol=1e-12), t


def test_prefill_full_window_is_causal_attention():
    """With the window covering everything, no selected blocks and the local gate saturated,
    the prefill is plain causal softmax attention."""
    rng = np.random.default_rng(9)
    B, H, L, dh = 1, 2, 40, 4
    q, k, v = (rng.standard_normal((B, H, L, dh)) for _ in range(3))
    idx = np.full((B, L, 1), 10**6)                 # out-of-range block: empty sparse stream
    gate = np.zeros((B, L, 3)); gate[..., 0] = 60.0
    got = osa.maba_sa_prefill_heads(q, k, v, None, None, np.zeros((B, H, L, dh)), idx, gate, window=L)
    s = np.einsum("bhtd,bhjd->bhtj", q, k) / 2.0
    s = np.where(np.tril(np.ones((L, L)))[None, None] > 0, s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    exp = np.einsum("bhtj,bhjd->bhtd", p / p.sum(-1, keepdims=True), v)
    assert np.allclose(got, exp, atol=1e-9)
