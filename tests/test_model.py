"""The full-model harness on the CPU (torch reference ops): the LatentCache serving loop
against the reference-style state passing of ``forward``/``step`` (model.py:207-270), on a
small configuration with both block kinds."""
import torch

from maba_sparse.model import MabaSparseForCausalLM, get_101m_config


def _small(seed=0):
    torch.manual_seed(seed)
    cfg = get_101m_config(dim=128, n_layers=4, n_heads=2, d_head=64, vocab_size=97, d_emb=16, d_c=32, d_idx=16,
                          intermediate_size=96, top_k=4, dist_lambda=0.1)
    return MabaSparseForCausalLM(cfg).init_normal(0.02).eval()


def test_101m_config_shape():
    m = MabaSparseForCausalLM(get_101m_config())
    kinds = [b.is_attention for b in m.layers]
    assert len(kinds) == 20 and sum(kinds) == 5 and kinds[3] and not kinds[0]     # 3:1 pattern
    n = sum(p.numel() for p in m.parameters())
    assert 90e6 < n < 110e6, n
    assert m.lm_head.weight is m.embeddings.in_emb.weight


def test_greedy_cache_loop_equals_state_passing():
    m = _small()
    ids = torch.randint(0, 97, (2, 150), generator=torch.Generator().manual_seed(1))
    steps = 12
    with torch.no_grad():
        got = m.generate_greedy(ids, steps)
        logits, states = m(ids)
        tok = logits[:, -1].argmax(-1, keepdim=True)
        ref = [tok]
        for _ in range(steps - 1):
            logits, states = m.step(tok, past_states=states)
            tok = logits[:, -1].argmax(-1, keepdim=True)
            ref.append(tok)
    assert torch.equal(got, torch.cat(ref, dim=1))


def test_parameter_names_follow_reference_model():
    """The names a reference state dict carries for these modules (model.py:62-205)."""
    m = MabaSparseForCausalLM(get_101m_config(n_layers=4))
    keys = set(m.state_dict())
    for k in ("embeddings.in_emb.weight", "embeddings.proj.weight", "final_norm.weight", "head_proj.weight",
              "lm_head.weight", "layers.0.norm1.weight", "layers.0.norm2.weight", "layers.0.res_gate1",
              "layers.0.res_gate2", "layers.0.ffn.w_gate.weight", "layers.0.ffn.w_up.weight",
              "layers.0.ffn.w_down.weight", "layers.0.mixer.q_proj.weight", "layers.0.mixer.conv_q.weight",
              "layers.0.mixer.gate_alpha.weight", "layers.3.mixer.kv_down_proj.weight",
              "layers.3.mixer.k_up_proj.weight", "layers.3.mixer.stream_gate.bias",
              "layers.3.mixer.indexer.q_idx_proj.weight"):
        assert k in keys, k
