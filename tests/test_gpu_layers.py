"""The callers on the GPU: each layer on cuda:0 (HIP ops) against the same layer on
the CPU (torch reference ops), over prefill + decode steps that cross 64-token
block boundaries.

Tolerances: fp32 modules 2e-3 (the north-star DGDA / sparse-attention bar);
indexer picks must agree wherever the CPU scores separate by more than 1e-4.
"""
import copy

import numpy as np
import pytest
import torch

from _helpers import assert_close, topk_agrees
from maba_sparse.layers import DGDALayer, DGIndexer, LatentCache, MabaSparseAttention

pytestmark = pytest.mark.gpu


def _x(B, T, D, seed):
    return torch.randn(B, T, D, generator=torch.Generator().manual_seed(seed))


def test_dgda_layer_gpu_matches_cpu(dev):
    torch.manual_seed(0)
    cpu = DGDALayer(dim=128, n_heads=2)
    gpu = copy.deepcopy(cpu).to(dev)
    x = _x(2, 150, 128, 1)
    with torch.no_grad():
        yc, Sc, csc = cpu(x[:, :140])
        yg, Sg, csg = gpu(x[:, :140].to(dev))
        assert_close(yg, yc.numpy(), 2e-3, 2e-3, "prefill out")
        assert_close(Sg, Sc.numpy(), 2e-3, 2e-3, "prefill state")
        for t in range(140, 150):
            yc, Sc, csc = cpu.step(x[:, t:t + 1], state=Sc, conv_state=csc)
            yg, Sg, csg = gpu.step(x[:, t:t + 1].to(dev), state=Sg, conv_state=csg)
            assert_close(yg, yc.numpy(), 2e-3, 2e-3, f"step {t}")
        assert_close(Sg, Sc.numpy(), 2e-3, 2e-3, "final state")


def test_indexer_layer_decode_gpu_matches_cpu(dev):
    torch.manual_seed(2)
    cpu = DGIndexer(dim=64, d_idx=64, top_k=8, dist_lambda=0.1).eval()
    gpu = copy.deepcopy(cpu).to(dev)
    x = _x(2, 700, 64, 3)
    with torch.no_grad():
        cpu(x[:, :600])
        gpu(x[:, :600].to(dev))
        checked = 0
        for t in range(600, 700):
            ic, cc, sc = cpu(x[:, t:t + 1], return_scores=True)
            ig, cg, _ = gpu(x[:, t:t + 1].to(dev), return_scores=True)
            assert_close(cg, cc.numpy(), 1e-5, 1e-5, f"centroids {t}")
            checked += topk_agrees(ig.cpu().numpy(), sc.double().numpy(), 8)
        assert checked > 150


@pytest.mark.parametrize("L0", [100, 1000])
def test_maba_sa_layer_decode_gpu_matches_cpu(dev, L0):
    torch.manual_seed(4)
    cpu = MabaSparseAttention(dim=128, n_heads=4, d_head=32, d_c=128, top_k=4).eval()
    gpu = copy.deepcopy(cpu).to(dev)
    x = _x(2, L0 + 70, 128, 5)
    with torch.no_grad():
        _, cc = cpu(x[:, :L0])
        _, cg = gpu(x[:, :L0].to(dev))
        for t in range(L0, L0 + 70):
            yc, cc = cpu(x[:, t:t + 1], past_c_kv=cc)
            yg, cg = gpu(x[:, t:t + 1].to(dev), past_c_kv=cg)
            assert_close(yg, yc.numpy(), 2e-3, 2e-3, f"decode {t}")


def test_maba_sa_layer_bf16_latent_cache(dev):
    """bf16 module on the GPU (MFMA decode path) with a preallocated LatentCache, against
    the fp32 CPU module: agreement to bf16 precision.  top_k exceeds the block count so
    the bf16 and fp32 indexers cannot pick different blocks."""
    torch.manual_seed(6)
    cpu = MabaSparseAttention(dim=128, n_heads=10, d_head=64, d_c=128, top_k=8).eval()
    gpu = copy.deepcopy(cpu).to(dev, torch.bfloat16)
    for p_c, p_g in zip(cpu.parameters(), gpu.parameters()):
        p_c.data.copy_(p_g.data.float().cpu())        # both see the same bf16-rounded weights
    x = _x(1, 400, 128, 7).bfloat16().float()
    with torch.no_grad():
        _, cc = cpu(x[:, :300])
        gpu(x[:, :300].to(dev, torch.bfloat16))
        cache = LatentCache(1, 512, 128, pool=64, device=dev, dtype=torch.bfloat16)
        cache.append(gpu.kv_down_proj(x[:, :300].to(dev, torch.bfloat16)))
        for t in range(300, 400):
            yc, cc = cpu(x[:, t:t + 1], past_c_kv=cc)
            yg = gpu.decode_step(x[:, t:t + 1].to(dev, torch.bfloat16), cache)
            ref = yc.numpy()
            err = np.abs(yg.float().cpu().numpy() - ref).max() / max(np.abs(ref).max(), 1e-6)
            assert err < 5e-2, (t, err)


def test_model_harness_gpu(dev):
    """The full-model harness on the GPU: fp32 prefill logits against the CPU model, the
    LatentCache serving loop against the reference-style state passing (same tokens), and a
    bf16 run through the fused prologue, prefill-attention and decode kernels."""
    from maba_sparse.model import MabaSparseForCausalLM, get_101m_config
    torch.manual_seed(0)
    cfg = get_101m_config(dim=128, n_layers=4, n_heads=2, d_head=64, vocab_size=97, d_emb=16, d_c=32, d_idx=16,
                          intermediate_size=96, top_k=4, dist_lambda=0.1)
    cpu = MabaSparseForCausalLM(cfg).init_normal(0.02).eval()
    gpu = copy.deepcopy(cpu).to(dev)
    ids = torch.randint(0, 97, (2, 300), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        lc, _ = cpu(ids)
        lg, states = gpu(ids.to(dev))
        scale = lc.abs().max().item()
        assert (lg.cpu() - lc).abs().max().item() <= 2e-3 * scale
        got = gpu.generate_greedy(ids.to(dev), 10)
        tok = lg[:, -1].argmax(-1, keepdim=True)
        ref = [tok]
        for _ in range(9):
            lg, states = gpu.step(tok, past_states=states)
            tok = lg[:, -1].argmax(-1, keepdim=True)
            ref.append(tok)
        assert torch.equal(got, torch.cat(ref, dim=1))
        bf = copy.deepcopy(cpu).to(dev, torch.bfloat16)
        lb, _ = bf(ids.to(dev))
        assert torch.isfinite(lb.float()).all()
        assert (lb.float().cpu() - lc).abs().max().item() <= 0.1 * scale
        toks = bf.generate_greedy(ids.to(dev), 6)
        assert toks.shape == (2, 6) and int(toks.min()) >= 0 and int(toks.max()) < 97


def test_model_fused_norm_prefill_matches_unfused(dev):
    """A bf16 model's ``forward`` on the HIP backend runs its norms, gated residuals and SwiGLU
    activations as HIP kernels: against the same model's torch elementwise path, for a whole
    prefill and for a prefill continued from the first half's states; ``last_only`` returns the
    last position's row of the full logits.  Tolerance: 3e-2 of the logits' largest magnitude (the
    two paths round the residual stream to bf16 at different points)."""
    from maba_sparse.model import MabaSparseForCausalLM, get_101m_config
    torch.manual_seed(3)
    cfg = get_101m_config(dim=128, n_layers=4, n_heads=2, d_head=64, vocab_size=97, d_emb=16, d_c=32, d_idx=16,
                          intermediate_size=96, top_k=4, dist_lambda=0.1)
    m = MabaSparseForCausalLM(cfg).init_normal(0.02).to(dev, torch.bfloat16).eval()
    ids = torch.randint(0, 97, (2, 300), generator=torch.Generator().manual_seed(4)).to(dev)
    with torch.no_grad():
        assert m._fused_norms_ok(m.embeddings(ids))
        lf, _ = m(ids)
        lf1, st = m(ids[:, :150])
        lf2, _ = m(ids[:, 150:], past_states=st)
        ll, _ = m(ids, last_only=True)
        m._fused_norms_ok = lambda x: False           # the torch elementwise path
        lu, _ = m(ids)
        lu1, su = m(ids[:, :150])
        lu2, _ = m(ids[:, 150:], past_states=su)
    scale = lu.float().abs().max().item()
    assert torch.isfinite(lf.float()).all()
    assert (lf.float() - lu.float()).abs().max().item() <= 3e-2 * scale
    assert (lf2.float() - lu2.float()).abs().max().item() <= 3e-2 * scale
    assert (torch.cat([lf1, lf2], dim=1).float() - lf.float()).abs().max().item() <= 3e-2 * scale
    assert ll.shape == (2, 1, 97)
    # the head GEMM over 2 rows or over 600 may sum in another order
    assert (ll[:, 0].float() - lf[:, -1].float()).abs().max().item() <= 1e-2 * scale
