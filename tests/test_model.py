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
