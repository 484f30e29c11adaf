"""The callers (maba_sparse/layers) on the CPU: call patterns into the dispatcher,
state/conv/cache carry across prefill and decode, and the fused MABA-SA decode
step against the dense streams at the same position.

Known answers from the reference's layer tests: the ``-0.75 ln 3`` indexer score
(test_indexer.py:143-164) and the causal block isolation (test_indexer.py:169-206).
"""
import math

import numpy as np
import pytest
import torch

from maba_sparse.layers import DGDALayer, DGIndexer, LatentCache, MabaSparseAttention
from maba_sparse.layers import dgda as dgda_mod
from oracle import dgda as odgda


def _x(B, T, D, seed, dtype=torch.float32):
    return torch.randn(B, T, D, generator=torch.Generator().manual_seed(seed)).to(dtype)


# ----------------------------------------------------------------------------- DGDA layer

REF_DGDA_PARAMS = {f"{n}.weight" for n in ("q_proj", "k_proj", "v_proj", "conv_q", "conv_k", "conv_v",
                                           "gate_alpha", "gate_erase", "gate_write", "o_proj")}


def test_dgda_parameter_names_match_reference():
    assert set(DGDALayer(dim=64, n_heads=2).state_dict()) == REF_DGDA_PARAMS


def test_dgda_call_pattern(monkeypatch):
    seen = {}

    def spy(**kw):
        seen.update(kw)
        B, H, L, _ = kw["q"].shape
        return torch.zeros(B, H, L, kw["v"].shape[-1]), torch.zeros(B, H, kw["q"].shape[-1], kw["v"].shape[-1])
    monkeypatch.setattr(dgda_mod, "dispatch_dgda_prefill", spy)
    torch.manual_seed(0)
    layer = DGDALayer(dim=64, n_heads=2)
    layer(_x(2, 9, 64, 0))
    assert set(seen) == {"q", "k", "v", "alpha", "b", "w", "chunk_size", "initial_state", "inversion_method",
                         "adaptive_tol", "log_alpha"}
    assert seen["chunk_size"] == 16 and seen["inversion_method"] == "adaptive" and seen["adaptive_tol"] == 7e-5
    # views, not copies: q/k/v keep the conv output's [B, H*d, T] storage (token stride 1),
    # the gates the projection's [B, T, H*d] storage (channel stride 1)
    assert seen["q"].shape == (2, 2, 9, 32) and seen["q"].stride()[2:] == (1, 9)
    assert seen["b"].stride()[1:] == (32, 64, 1)
    assert (seen["log_alpha"] >= -14.0).all()
    assert torch.allclose(seen["alpha"], seen["log_alpha"].exp())
    n = seen["k"].norm(dim=-1)          # k / (|k| + eps): unit norm up to eps / |k|
    assert (n <= 1.0).all() and (n > 0.99).all()


def test_dgda_layer_matches_oracle_recurrence(monkeypatch):
    """The layer's op inputs through the float64 token-loop oracle give the layer's output."""
    captured = {}
    real = dgda_mod.dispatch_dgda_prefill

    def spy(**kw):
        captured.update(kw)
        return real(**kw)
    monkeypatch.setattr(dgda_mod, "dispatch_dgda_prefill", spy)
    torch.manual_seed(0)
    layer = DGDALayer(dim=64, n_heads=2).double()
    layer.inversion_method = "exact"   # the cpu backend's chunked form with the exact triangular solve
    y, S, _ = layer(_x(1, 30, 64, 1, torch.float64))
    f = lambda t: t.detach().numpy()  # noqa: E731
    eo, eS = odgda.dgda_prefill_seq(f(captured["q"]), f(captured["k"]), f(captured["v"]), alpha=f(captured["alpha"]),
                                    b=f(captured["b"]), w=f(captured["w"]))
    assert np.allclose(f(S), eS, atol=1e-10)
    o = torch.from_numpy(eo).transpose(1, 2).reshape(1, 30, 64)
    assert torch.allclose(y, layer.o_proj(o), atol=1e-10)


def test_dgda_prefill_then_steps_equals_one_prefill():
    torch.manual_seed(1)
    layer = DGDALayer(dim=64, n_heads=2).double()
    layer.inversion_method = "exact"   # chunked prefill with the exact solve: consistent to fp64 rounding
    x = _x(2, 20, 64, 2, torch.float64)
    y_all, S_all, _ = layer(x)
    y, S, cs = layer(x[:, :13])
    outs = [y]
    for t in range(13, 20):
        yt, S, cs = layer.step(x[:, t:t + 1], state=S, conv_state=cs)
        outs.append(yt)
    assert torch.allclose(torch.cat(outs, 1), y_all, atol=1e-10)
    assert torch.allclose(S, S_all, atol=1e-10)


def test_dgda_split_prefill_and_conv_state_forms():
    torch.manual_seed(2)
    layer = DGDALayer(dim=64, n_heads=2).double()
    layer.inversion_method = "exact"   # chunked prefill with the exact solve: consistent to fp64 rounding
    x = _x(1, 25, 64, 3, torch.float64)
    y_all, S_all, _ = layer(x)
    y1, S1, cs = layer(x[:, :11])
    for form in (cs, tuple(cs), cs.as_tensor(), cs.as_tensor().reshape(1, -1, 3)):
        y2, S2, _ = layer(x[:, 11:], state=S1, conv_state=form)
        assert torch.allclose(torch.cat([y1, y2], 1), y_all, atol=1e-10)
        assert torch.allclose(S2, S_all, atol=1e-10)
    assert cs.shape == torch.Size([1, 3, 64, 3])


def test_dgda_empty_sequence():
    layer = DGDALayer(dim=64, n_heads=2)
    y, S, cs = layer(torch.zeros(2, 0, 64))
    assert y.shape == (2, 0, 64) and S.shape == (2, 2, 32, 32) and (S == 0).all() and cs.shape[1] == 3


# ----------------------------------------------------------------------------- indexer layer

def test_indexer_log_distance_known_answer():
    ix = DGIndexer(dim=64, d_idx=32, block_size=64, dist_lambda=0.75).eval()
    with torch.no_grad():
        ix.q_idx_proj.weight.zero_()
        ix.k_idx_proj.weight.zero_()
    _, _, sc = ix(torch.zeros(1, 256, 64), return_scores=True)
    assert math.isclose(sc[0, 192, 1].item(), -0.75 * math.log(3.0), rel_tol=1e-5)


def test_indexer_causal_block_isolation():
    ix = DGIndexer(dim=64, d_idx=32, block_size=64, top_k=8, dist_lambda=0.5).eval()
    idx, _, sc = ix(torch.randn(1, 512, 64), return_scores=True)
    for t in [0, 31, 63, 64, 127, 250, 511]:
        qb = t // 64
        assert torch.isinf(sc[0, t, qb + 1:]).all() and torch.isfinite(sc[0, t, : qb + 1]).all()
        assert (idx[0, t, : qb + 1] <= qb).all()


def test_indexer_decode_cache_equals_full_recompute():
    """Prefill 150 keys, then 100 decode steps through the cache (block completions at
    192 and 256): each step's centroids and picks equal the stateless past_k_idx branch."""
    torch.manual_seed(3)
    ix = DGIndexer(dim=32, d_idx=16, block_size=64, top_k=4, dist_lambda=0.3).eval()
    x = torch.randn(2, 250, 32)
    ix(x[:, :150])
    for t in range(150, 250):
        idx, c = ix(x[:, t:t + 1])
        ref_idx, ref_c = DGIndexer.forward(ix, x[:, t:t + 1], past_k_idx=ix.k_idx_proj(x[:, :t]))
        assert torch.allclose(c, ref_c, atol=1e-6), t
        assert torch.equal(idx, ref_idx), t
        assert ix._cached_k_idx.shape[1] == t + 1


def test_indexer_past_centroids_branch():
    torch.manual_seed(4)
    ix = DGIndexer(dim=32, d_idx=16).eval()
    pc = torch.randn(2, 5, 16)
    idx, c = ix(torch.randn(2, 1, 32), past_centroids=pc)
    assert c.shape == (2, 6, 16) and torch.equal(c[:, :5], pc) and idx.shape == (2, 1, 6)


# ----------------------------------------------------------------------------- MABA-SA layer

def _sa(seed=5, **kw):
    torch.manual_seed(seed)
    return MabaSparseAttention(dim=64, n_heads=2, d_head=16, d_c=32, top_k=3, **kw).eval()


@pytest.mark.parametrize("T", [40, 63, 64, 200, 333])
def test_sa_fused_decode_equals_dense_last_row(T):
    """The latent-space fused decode of token T-1 equals the dense streams' last row."""
    layer = _sa()
    x = _x(2, T, 64, T)
    with torch.no_grad():
        y_dense, c_full = layer(x)
        layer.reset_cache()
        _, c_prev = layer(x[:, : T - 1])
        y_dec, c2 = layer(x[:, T - 1:], past_c_kv=c_prev)
    assert torch.allclose(c2, c_full, atol=1e-6)
    assert torch.allclose(y_dec[:, 0], y_dense[:, -1], rtol=1e-4, atol=1e-5)


def test_sa_decode_loop_with_latent_cache():
    """decode_step over a preallocated LatentCache equals forward(past_c_kv) step by step,
    across HCA block completions."""
    layer_a, layer_b = _sa(6), _sa(6)
    x = _x(1, 200, 64, 7)
    with torch.no_grad():
        _, c = layer_a(x[:, :120])
        layer_b(x[:, :120])
        cache = LatentCache(1, 256, 32, pool=64)
        cache.append(layer_b.kv_down_proj(x[:, :120]))
        for t in range(120, 200):
            ya, c = layer_a(x[:, t:t + 1], past_c_kv=c)
            yb = layer_b.decode_step(x[:, t:t + 1], cache)
            assert torch.allclose(ya, yb, atol=1e-6), t
        assert cache.n == 200 and cache.nh == 3
        assert torch.allclose(cache.c[:, :200], c, atol=1e-6)


def test_sa_ablation_no_hca_uses_dense_path():
    layer = _sa(ablation_mode="no_hca")
    x = _x(1, 70, 64, 8)
    with torch.no_grad():
        y, c = layer(x)
        y1, _ = layer(x[:, 69:], past_c_kv=c[:, :69])
    assert y.shape == (1, 70, 64) and y1.shape == (1, 1, 64)


def test_prefill_form_follows_selection_sharing():
    """The fused prefill takes the head-space union kernel when 16 consecutive queries share
    their blocks and the latent kernel when their selections scatter (the union of 16 query
    rows is counted from the indices)."""
    from maba_sparse.layers import MabaSparseAttention
    layer = MabaSparseAttention(dim=64, n_heads=2, d_head=32, d_c=32, d_idx=16, top_k=8)
    B, Lq, K = 2, 64, 8
    shared = torch.arange(K).repeat(B, Lq, 1)                            # every query the same 8 blocks
    assert layer._prefill_form(shared) == "heads"
    g = torch.Generator().manual_seed(0)
    scattered = torch.stack([torch.randperm(4096, generator=g)[:K] for _ in range(B * Lq)]).view(B, Lq, K)
    assert layer._prefill_form(scattered) == "latent"
    assert layer._prefill_form(shared[:, :1]) == "heads"                 # one row for all queries
    layer.prefill_form = "latent"
    assert layer._prefill_form(shared) == "latent"
