"""Weight-derived caches of the decode paths (stacked projections, fp32 head views, gate
sigmoids) follow weight updates, and the stacked MABA-SA projection hands the indexer an
8-aligned query view (the bf16 MFMA decode scoring needs 16-byte aligned query rows)."""
import copy

import torch

from maba_sparse.layers import DGDALayer, LatentCache, MabaSparseAttention


def _sa_pair(seed=0):
    torch.manual_seed(seed)
    layer = MabaSparseAttention(dim=64, n_heads=2, d_head=32, d_c=32, d_idx=16, top_k=4).eval()
    return layer


def _decode(layer, x, prefix):
    cache = LatentCache(x.shape[0], 256, layer.d_c, pool=64)
    with torch.no_grad():
        layer(prefix)
        cache.append(layer.kv_down_proj(prefix))
        return layer.decode_step(x, cache)


def test_stacked_projection_query_is_aligned():
    layer = _sa_pair()
    x = torch.randn(3, 1, 64)
    with torch.no_grad():
        q, c_new, qi, ki, gl = layer._token_projections(x)
    assert qi.stride(0) % 8 == 0 and qi.stride(1) % 8 == 0
    assert qi.storage_offset() == 0
    with torch.no_grad():
        assert torch.allclose(qi, layer.indexer.q_idx_proj(x), atol=1e-6)
        assert torch.allclose(ki, layer.indexer.k_idx_proj(x), atol=1e-6)
        assert torch.allclose(q, layer.q_proj(x), atol=1e-6)
        assert torch.allclose(c_new, layer.kv_down_proj(x), atol=1e-6)
        assert torch.allclose(gl, layer.stream_gate(x), atol=1e-6)


def test_maba_sa_data_write_then_clear():
    layer = _sa_pair()
    prefix, x = torch.randn(2, 100, 64), torch.randn(2, 1, 64)
    _decode(layer, x, prefix)                                   # builds the caches
    with torch.no_grad():
        for p in (layer.q_proj.weight, layer.k_up_proj.weight, layer.v_up_proj.weight, layer.stream_gate.weight):
            p.data.mul_(1.7)                                    # no version bump
    layer.clear_weight_caches()
    fresh = copy.deepcopy(layer)
    fresh.clear_weight_caches()
    assert torch.allclose(_decode(layer, x, prefix), _decode(fresh, x, prefix), atol=1e-6)


def test_in_place_update_rebuilds_without_clear():
    layer = _sa_pair(1)
    prefix, x = torch.randn(2, 70, 64), torch.randn(2, 1, 64)
    _decode(layer, x, prefix)
    with torch.no_grad():
        layer.q_proj.weight.mul_(0.5)                           # bumps _version
        layer.v_up_proj.weight.add_(0.01)
    fresh = copy.deepcopy(layer)
    fresh.clear_weight_caches()
    assert torch.allclose(_decode(layer, x, prefix), _decode(fresh, x, prefix), atol=1e-6)


def test_load_state_dict_clears():
    layer = _sa_pair(2)
    other = _sa_pair(3)
    prefix, x = torch.randn(1, 80, 64), torch.randn(1, 1, 64)
    _decode(layer, x, prefix)
    layer.load_state_dict(other.state_dict())
    assert not [k for k in layer.__dict__ if k.startswith("_wcache_")]
    assert torch.allclose(_decode(layer, x, prefix), _decode(other, x, prefix), atol=1e-6)


def test_dgda_stack_follows_data_write():
    torch.manual_seed(4)
    layer = DGDALayer(dim=64, n_heads=1).eval()
    x = torch.randn(1, 1, 64)
    with torch.no_grad():
        layer.step(x)
        layer.gate_alpha.weight.data.mul_(-2.0)
        layer.clear_weight_caches()
        fresh = copy.deepcopy(layer)
        assert torch.allclose(layer.step(x)[0], fresh.step(x)[0], atol=1e-6)


def test_generate_greedy_sees_data_writes():
    from maba_sparse.model import MabaSparseForCausalLM, get_101m_config
    torch.manual_seed(0)
    cfg = get_101m_config(dim=64, n_layers=4, n_heads=1, d_head=64, vocab_size=50, d_emb=16, d_c=32, d_idx=16,
                          intermediate_size=48, top_k=4)
    model = MabaSparseForCausalLM(cfg).init_normal(0.02).eval()
    ids = torch.randint(0, 50, (2, 70), generator=torch.Generator().manual_seed(1))
    model.generate_greedy(ids, 3)                              # fills every weight cache
    with torch.no_grad():
        for blk in model.layers:
            blk.ffn.w_gate.weight.data.mul_(3.0)
            blk.res_gate1.data.fill_(-1.0)
            if blk.is_attention:
                blk.mixer.q_proj.weight.data.mul_(2.0)
            else:
                blk.mixer.q_proj.weight.data.mul_(2.0)
    fresh = copy.deepcopy(model)
    fresh.clear_weight_caches()
    a_tok, a_lg = model.generate_greedy(ids, 4, return_logits=True)
    b_tok, b_lg = fresh.generate_greedy(ids, 4, return_logits=True)
    assert torch.equal(a_tok, b_tok)
    assert torch.allclose(a_lg, b_lg, atol=1e-6)
