"""BASELINE configs 3 and 4 at their full size on the GPU, against the float64 oracle.

Config 3: 1,000,000 latent keys x d_c = 128 per sequence (B = 8, bf16 ~ N(0,1)) with one
planted key of 8x norm at a seeded position; 64-token block centroids 0.5 (mean + max);
ten 128-dim query heads; decode scores with lambda = 0.1 log(1 + distance); top-32.
Config 4: the fused MABA-SA decode step over the same cache at L = 1,000,000, H = 10,
d_head = 64, W_k / W_v ~ N(0, 0.02), gate logits ~ N(0,1), with the config-3 selections
as per-head index sets [8, 10, 32] and as one shared set per sequence [8, 1, 32].

The oracle sees only the stored bf16 values (as float64) and computes its own block
centroids and HCA means, one sequence at a time.  Tolerances:
- centroids: the bf16 rounding of the exact value, 2^-8 relative (one ulp);
- scores 1e-5 relative + 1e-4 absolute; selections bit-exact wherever the reference's score
  gap exceeds 1e-4 (the north-star criterion; 75 of the 80 rows here), and on every row a
  valid top-32 of the reference scores up to 1e-4;
- attention output rtol = atol = 2e-3, and each stream alone (the gate
  saturated on it) within 2e-3 of that stream's largest output magnitude: the kernel reads
  the bf16 means the cache stores, the oracle exact means.
"""
import math

import numpy as np
import pytest
import torch

from _helpers import assert_close, to_np, topk_agrees, topk_is_valid
from oracle import indexer as oidx
from oracle import sparse_attn as osa

pytestmark = pytest.mark.gpu

B, L, DC, HQ, H, DH, K, LAM = 8, 1_000_000, 128, 10, 10, 64, 32, 0.1
NB = (L + 63) // 64
ALIGNED_HEAD = 3


def _hip():
    from maba_sparse.kernels import hip_backend
    return hip_backend


@pytest.fixture(scope="module")
def cache():
    import conftest
    if not conftest.gpu_available():
        pytest.skip("no ROCm GPU")
    dev = torch.device("cuda:0")
    print(f"\nconfig 3/4 cache: B={B} L={L} d_c={DC}", flush=True)
    gen = torch.Generator(device=dev).manual_seed(2024)
    c_kv = torch.randn(B, L, DC, device=dev, generator=gen, dtype=torch.bfloat16)
    pos = torch.randint(0, L, (B,), generator=torch.Generator().manual_seed(3))
    for b in range(B):      # one salient token per sequence, norm x8
        c_kv[b, pos[b]] *= 8
    cent = _hip().hip_compute_centroids(c_kv, block_size=64)
    hca = _hip().hip_hca_pool(c_kv, pool=64)
    g = torch.Generator().manual_seed(5)
    q_idx = torch.randn(B, HQ, DC, generator=g)
    for b in range(B):      # head 3 points at the planted key
        p = c_kv[b, pos[b]].float().cpu()
        q_idx[b, ALIGNED_HEAD] = p / p.norm() * math.sqrt(DC)
    q_idx = q_idx.bfloat16().to(dev)
    torch.cuda.synchronize()
    return dict(dev=dev, c_kv=c_kv, pos=pos, cent=cent, hca=hca, q_idx=q_idx)


def _seq(c_kv, b):
    """Sequence b of the cache as float64 on the host (1 GB)."""
    return c_kv[b:b + 1].double().cpu().numpy()


def test_config3_centroids_1M(cache):
    cent = cache["cent"]
    assert cent.shape == (B, NB, DC) and cent.dtype == torch.bfloat16
    for b in range(B):
        exp = oidx.compute_centroids(_seq(cache["c_kv"], b), 64)[0]
        got = cent[b].double().cpu().numpy()
        err = np.abs(got - exp)
        bound = (2.0 ** -8 + 1e-5) * np.abs(exp) + 1e-6      # half an ulp plus fp32 slack
        bad = err > bound
        assert not bad.any(), f"b={b}: {bad.sum()} centroids off by more than one bf16 ulp (max err {err.max():.3e})"
        blk = int(cache["pos"][b]) // 64
        assert np.abs(exp[blk]).max() > 8.0, "the planted key dominates its block's centroid"


def test_config3_decode_topk_1M(cache):
    q_idx, cent = cache["q_idx"], cache["cent"]
    idx, sc = _hip().hip_index_topk_decode(q_idx, cent, lambda_dist=LAM, top_k=K, return_scores=True)
    assert idx.shape == (B, HQ, K) and idx.dtype == torch.long
    ref = oidx.decode_scores(to_np(q_idx), to_np(cent), LAM)       # scores of the stored bf16 centroids
    assert_close(sc, ref, 1e-5, 1e-4, "decode scores at 1M")
    checked = topk_agrees(idx.cpu().numpy(), ref, K, gap=1e-4)      # bit-exact where the gap exceeds 1e-4
    assert checked >= B * HQ * 3 // 4, f"only {checked} of {B * HQ} rows separate by more than 1e-4"
    topk_is_valid(idx.cpu().numpy(), ref, 1e-4)                      # every row, near-ties included
    for b in range(B):
        assert idx[b, ALIGNED_HEAD, 0].item() == int(cache["pos"][b]) // 64, f"b={b}: planted block not first"
    cache["idx"] = idx


def _oracle_streams(cache, q, Wk, Wv, idx_sets):
    """Per-stream oracle outputs [B, H, dh]: local, sparse (one per index-set variant), HCA."""
    ol = np.zeros((B, H, DH))
    oh = np.zeros((B, H, DH))
    os_ = [np.zeros((B, H, DH)) for _ in idx_sets]
    qn, Wkn, Wvn = to_np(q), to_np(Wk), to_np(Wv)
    for b in range(B):
        c_b = _seq(cache["c_kv"], b)
        means = osa.hca_means(c_b, L, 64)
        ol[b] = osa.local_stream(qn[b:b + 1], c_b, Wkn, Wvn, L)[0]
        oh[b] = osa.hca_stream(qn[b:b + 1], c_b, Wkn, Wvn, L, 64, means=means)[0]
        for v, ix in enumerate(idx_sets):
            os_[v][b] = osa.sparse_stream(qn[b:b + 1], c_b, Wkn, Wvn, ix[b:b + 1], L)[0]
    return ol, os_, oh


def test_config4_maba_sa_decode_1M(cache):
    dev = cache["dev"]
    if "idx" not in cache:
        cache["idx"] = _hip().hip_index_topk_decode(cache["q_idx"], cache["cent"], lambda_dist=LAM, top_k=K)
    idx_per = cache["idx"]                          # [8, 10, 32] per-head sets from config 3
    idx_sh = idx_per[:, :1].contiguous()           # [8, 1, 32] one set per sequence
    g = torch.Generator().manual_seed(9)
    Wk = (torch.randn(H * DH, DC, generator=g) * 0.02).bfloat16().float()
    Wv = (torch.randn(H * DH, DC, generator=g) * 0.02).bfloat16().float()
    q = torch.randn(B, H, DH, generator=g)
    gate = torch.randn(B, 3, generator=g)
    q_lat = torch.einsum("bhd,hdc->bhc", q, Wk.view(H, DH, DC)).to(dev)      # W_k,h^T q_h
    Wv_h = Wv.view(H, DH, DC)
    scale = 1.0 / math.sqrt(DH)
    print("config 4: oracle streams", flush=True)
    ol, os_list, oh = _oracle_streams(cache, q, Wk, Wv, [to_np(idx_per).astype(np.int64),
                                                         to_np(idx_sh).astype(np.int64)])

    def run(ix, gl):
        z = _hip().hip_maba_sa_decode(q_lat, cache["c_kv"], cache["hca"], ix, gl.to(dev), L=L, scale=scale)
        return torch.einsum("bhc,hdc->bhd", z.cpu(), Wv_h).double().numpy()

    for ix, os_, what in ((idx_per, os_list[0], "per-head sets"), (idx_sh, os_list[1], "shared sets")):
        g4 = to_np(gate)[:, None, None, :]
        exp = osa.superposition(ol[:, :, None], os_[:, :, None], oh[:, :, None], gate_logits=g4)[:, :, 0]
        assert_close(run(ix, gate), exp, 2e-3, 2e-3, f"config 4 output, {what}")
        for s, ref in enumerate((ol, os_, oh)):          # each stream alone: gate saturated on it
            gl = torch.full((B, 3), -60.0)
            gl[:, s] = 60.0
            got = run(ix, gl)
            err = np.abs(got - ref).max() / np.abs(ref).max()
            assert err <= 2e-3, f"config 4 stream {s} alone ({what}): normwise error {err:.2e}"
