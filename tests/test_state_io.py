"""The persisted decode state (maba_sparse/state_io.py) on the CPU: a prefill's state written
to a file and read into a second copy of the model continues exactly like the original, for
several decode steps across a 64-token block boundary; mismatched files are refused."""
import copy

import pytest
import torch

from maba_sparse.model import MabaSparseForCausalLM, get_101m_config
from maba_sparse.state_io import load_decode_state, save_decode_state


def _small(seed=0):
    torch.manual_seed(seed)
    cfg = get_101m_config(dim=128, n_layers=4, n_heads=2, d_head=64, vocab_size=97, d_emb=16, d_c=32, d_idx=16,
                          intermediate_size=96, top_k=4, dist_lambda=0.1)
    return MabaSparseForCausalLM(cfg).init_normal(0.02).eval()


def test_saved_state_resumes_exactly(tmp_path):
    m = _small()
    ids = torch.randint(0, 97, (2, 190), generator=torch.Generator().manual_seed(3))
    path = str(tmp_path / "state.safetensors")
    with torch.no_grad():
        logits, states = m(ids)
        save_decode_state(m, states, path)
        m2 = copy.deepcopy(m)
        for layer in m2.layers:                # a fresh copy holds no caches
            if layer.is_attention:
                layer.mixer.reset_cache()
        states2 = load_decode_state(m2, path)
        tok = logits[:, -1].argmax(-1, keepdim=True)
        for _ in range(5):                     # positions 190..194 cross the block edge at 192
            la, states = m.step(tok, past_states=states)
            lb, states2 = m2.step(tok, past_states=states2)
            assert torch.equal(la, lb)
            tok = la[:, -1].argmax(-1, keepdim=True)


def test_resume_without_indexer_keys_differs(tmp_path):
    """Why the indexer keys are part of the format: the latent rows alone (the reference's
    ``past_states``) leave the resumed indexer without its history, and the next step differs."""
    m = _small()
    ids = torch.randint(0, 97, (2, 190), generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        logits, states = m(ids)
        m2 = copy.deepcopy(m)
        for layer in m2.layers:
            if layer.is_attention:
                layer.mixer.reset_cache()
        tok = logits[:, -1].argmax(-1, keepdim=True)
        la, _ = m.step(tok, past_states=states)
        lb, _ = m2.step(tok, past_states=states)
    assert not torch.equal(la, lb)


def test_load_refuses_other_files(tmp_path):
    from safetensors.torch import save_file
    m = _small()
    bad = str(tmp_path / "bad.safetensors")
    save_file({"x": torch.zeros(1)}, bad, metadata={"format": "something-else"})
    with pytest.raises(ValueError, match="not a maba-decode-state"):
        load_decode_state(m, bad)
    ids = torch.randint(0, 97, (1, 70), generator=torch.Generator().manual_seed(5))
    path = str(tmp_path / "s.safetensors")
    with torch.no_grad():
        _, states = m(ids)
    save_decode_state(m, states, path)
    other = MabaSparseForCausalLM(get_101m_config(dim=128, n_layers=3, n_heads=2, d_head=64, vocab_size=97, d_emb=16,
                                                  d_c=32, d_idx=16, intermediate_size=96, top_k=4)).eval()
    with pytest.raises(ValueError, match="block pattern"):
        load_decode_state(other, path)
