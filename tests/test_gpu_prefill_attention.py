"""MABA-SA prefill streams on the GPU (``maba_hip_maba_sa_prefill``) against the float64
oracle (``oracle.sparse_attn.maba_sa_prefill_heads``, pinned against the decode oracle at
every prefix length) and, at a longer shape, against the torch reference op on the GPU.

Tolerance: rtol = atol = 2e-3 (the north-star sparse-attention bar) on bf16 inputs with
fp32 accumulation; the bf16 layer against its own dense torch path: 3e-2 of the output's
largest magnitude (the dense path rounds its scores and probabilities to bf16).
"""
import copy

import numpy as np
import pytest
import torch

from _helpers import assert_close, to_np
from oracle import sparse_attn as osa

pytestmark = pytest.mark.gpu


def _hip():
    from maba_sparse.kernels import hip_backend
    return hip_backend


def _case(B, H, Lq, Lkv, dh, K, seed, shared=False, gate4=False, dup=False):
    g = torch.Generator().manual_seed(seed)
    bf = lambda *s: torch.randn(*s, generator=g).bfloat16()  # noqa: E731
    q, k, v = bf(B, H, Lq, dh), bf(B, H, Lkv, dh), bf(B, H, Lkv, dh)
    nc = Lkv // 64
    kh, vh = (bf(B, H, nc, dh), bf(B, H, nc, dh)) if nc > 0 else (None, None)
    off = Lkv - Lq
    n_early = max(0, min(Lq, 63 - off))
    early = bf(B, H, n_early, dh) if n_early > 0 else None
    nb = (Lkv + 63) // 64
    rows = 1 if shared else Lq
    idx = torch.randint(0, nb, (B, rows, K), generator=g)
    idx[:, :, 0] = -1 if K > 2 else idx[:, :, 0]             # an empty slot (ignored)
    if dup and K > 2:
        idx[:, ::3, 2] = idx[:, ::3, 1]                        # repeated blocks count twice
    gate = torch.randn(B, H, Lq, 3, generator=g) if gate4 else torch.randn(B, Lq, 3, generator=g)
    return q, k, v, kh, vh, early, idx, gate


@pytest.mark.parametrize("B,H,Lq,Lkv,dh,K,window,n_sink,shared,gate4,dup", [
    (2, 3, 150, 150, 64, 4, 128, 4, False, False, True),   # early rows, one complete mean, repeats
    (1, 2, 77, 300, 64, 8, 40, 2, False, True, False),     # a past, per-head gates, narrow window
    (2, 2, 64, 64, 32, 3, 16, 0, True, False, False),      # d_head 32, one index row for all queries
    (1, 2, 40, 40, 128, 2, 128, 4, False, False, False),   # d_head 128, no complete block: all early
    (1, 4, 1000, 1000, 64, 32, 128, 4, False, False, True),
    (1, 2, 700, 2000, 64, 16, 300, 70, False, False, False),  # sinks wider than one tile
])
def test_maba_sa_prefill(dev, B, H, Lq, Lkv, dh, K, window, n_sink, shared, gate4, dup):
    q, k, v, kh, vh, early, idx, gate = _case(B, H, Lq, Lkv, dh, K, Lq + Lkv + dh, shared, gate4, dup)
    d = lambda t: None if t is None else t.to(dev)  # noqa: E731
    out = _hip().hip_maba_sa_prefill(d(q), d(k), d(v), d(kh), d(vh), d(early), d(idx), d(gate),
                                     scale=dh ** -0.5, window=window, n_sink=n_sink, out_dtype=torch.float32)
    exp = osa.maba_sa_prefill_heads(to_np(q), to_np(k), to_np(v), to_np(kh), to_np(vh), to_np(early), idx.numpy(),
                                    to_np(gate), window=window, n_sink=n_sink, scale=dh ** -0.5)
    assert_close(out, exp, 2e-3, 2e-3, "maba_sa_prefill")
    out_bf = _hip().hip_maba_sa_prefill(d(q), d(k), d(v), d(kh), d(vh), d(early), d(idx), d(gate),
                                        scale=dh ** -0.5, window=window, n_sink=n_sink)
    assert out_bf.dtype == torch.bfloat16
    assert torch.equal(out_bf, out.bfloat16())   # the bf16 output is the fp32 result rounded once


def test_maba_sa_prefill_long_against_torch_reference(dev):
    """4,096 queries over their own 4,096 keys with 32 causal blocks each, against the torch
    reference op on the GPU (dense masks, fp32)."""
    from maba_sparse.kernels import common as C
    B, H, L, dh, K = 1, 4, 4096, 64, 32
    q, k, v, kh, vh, early, _, gate = _case(B, H, L, L, dh, K, 5)
    g = torch.Generator().manual_seed(6)
    pos_blk = torch.arange(L) // 64
    idx = (torch.rand(B, L, K, generator=g) * (pos_blk[None, :, None] + 1).float()).long()   # causal blocks
    d = lambda t: None if t is None else t.to(dev)  # noqa: E731
    args = [d(t) for t in (q, k, v, kh, vh, early, idx, gate)]
    out = _hip().hip_maba_sa_prefill(*args, scale=0.125, out_dtype=torch.float32)
    ref = C.ref_maba_sa_prefill(*args, scale=0.125, out_dtype=torch.float32)
    assert_close(out, to_np(ref), 2e-3, 2e-3, "maba_sa_prefill 4k")


def test_bench_row_32k_both_kernels_vs_oracle(dev):
    """The bench row `maba_sa_prefill_32k` at its own shape and inputs: B=1, H=10, d_head 64,
    d_c 128, 32,768 queries over their own keys, top-32 causal blocks from the HIP prefill
    top-k (lambda 0.5, recency-biased, about 5 K distinct blocks per 16 queries), 512 means.
    Both kernels, composed as the bench composes them (the head-space kernel over bf16
    up-projected keys, values and means, fp32 early rows; the latent kernel over the bf16 latent
    rows and their means, then W_v,h), at rows spread over the sequence (the first, the last
    early row, block edges, deep rows), against the oracle's decode at that position
    (float64, the same bf16 weights), rtol = atol = 2e-3."""
    hb = _hip()
    B, H, L, dh, dc, K = 1, 10, 32768, 64, 128, 32
    g = torch.Generator(device=dev).manual_seed(21)
    bf = lambda *sh: torch.randn(*sh, device=dev, generator=g, dtype=torch.bfloat16)  # noqa: E731
    q, c = bf(B, H, L, dh), bf(B, L, dc)
    Wkb = (torch.randn(H * dh, dc, device=dev, generator=g) * dc ** -0.5).bfloat16()
    Wvb = (torch.randn(H * dh, dc, device=dev, generator=g) * dc ** -0.5).bfloat16()
    gate = torch.randn(B, L, 3, device=dev, generator=g)
    idx = hb.hip_index_topk(bf(B, L, 64), bf(B, L // 64, 64), lambda_dist=0.5, top_k=K, block_size=64)
    heads = lambda t, n: t.view(B, n, H, dh).transpose(1, 2)  # noqa: E731
    with torch.no_grad():
        k, v = heads(c @ Wkb.t(), L), heads(c @ Wvb.t(), L)
        means = c.reshape(B, L // 64, 64, dc).float().mean(dim=2).bfloat16()
        kh, vh = heads(means @ Wkb.t(), L // 64), heads(means @ Wvb.t(), L // 64)
        cnt = torch.arange(1, 64, device=dev, dtype=torch.float32).view(1, -1, 1)
        # early rows in fp32: at row 0 the output is (up to the gate) this row itself, so a bf16
        # rounding of it alone would exceed the tolerance
        early = heads((torch.cumsum(c[:, :63].float(), dim=1) / cnt) @ Wvb.float().t(), 63)
        o_heads = hb.hip_maba_sa_prefill(q, k, v, kh, vh, early, idx, gate, scale=dh ** -0.5,
                                         out_dtype=torch.float32)
        Wk_h, Wv_h = Wkb.float().view(H, dh, dc), Wvb.float().view(H, dh, dc)
        q_lat = torch.einsum("bhtd,hdc->bthc", q.float(), Wk_h).contiguous()
        z = hb.hip_maba_sa_prefill_latent(q_lat, c, hb.hip_hca_pool(c, pool=64), idx, gate, scale=dh ** -0.5)
        o_latent = torch.einsum("bthc,hdc->bhtd", z, Wv_h)
        torch.cuda.synchronize()
    Wk, Wv = to_np(Wkb), to_np(Wvb)
    for t in (0, 62, 63, 64, 4095, 16384 + 33, L - 1):
        exp = osa.maba_sa_decode(to_np(q[:, :, t]), to_np(c[:, : t + 1]), Wk, Wv, idx[:, t:t + 1].cpu().numpy(),
                                 to_np(gate[:, t]), L=t + 1)
        assert_close(o_heads[:, :, t], exp, 2e-3, 2e-3, f"head-space kernel row {t}")
        assert_close(o_latent[:, :, t], exp, 2e-3, 2e-3, f"latent kernel row {t}")


@pytest.mark.parametrize("form", ["latent", "heads", "auto"])
def test_layer_prefill_fused_matches_dense_path(dev, form):
    """The bf16 MabaSparseAttention prefill through either HIP kernel (the latent form, the
    head-space union form, or the layer's choice between them) against the same layer's dense
    torch path."""
    from maba_sparse.layers import MabaSparseAttention
    torch.manual_seed(8)
    layer = MabaSparseAttention(dim=256, n_heads=4, d_head=64, d_c=64, d_idx=32, top_k=8,
                                dist_lambda=0.1).to(dev, torch.bfloat16).eval()
    layer.prefill_form = form
    dense = copy.deepcopy(layer)
    dense._prefill_fusable = lambda *a: False
    x = torch.randn(2, 700, 256, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        yf, cf = layer(x)
        yd, cd = dense(x)
        assert torch.equal(cf, cd)
        err = (yf.float() - yd.float()).abs().max().item()
        assert err <= 3e-2 * yd.float().abs().max().item(), err


@pytest.mark.parametrize("Lq,Lkv,window,n_sink,empty_sparse", [
    (1, 1, 128, 4, False),      # one token
    (1, 500, 128, 4, False),    # one query over a past: a decode step
    (50, 200, 0, 0, False),     # no local keys at all: the local stream contributes 0
    (40, 100, 16, 200, True),   # sinks wider than the sequence; every index slot empty
])
def test_maba_sa_prefill_edges(dev, Lq, Lkv, window, n_sink, empty_sparse):
    B, H, dh, K = 2, 2, 64, 4
    q, k, v, kh, vh, early, idx, gate = _case(B, H, Lq, Lkv, dh, K, Lq * 7 + Lkv)
    if empty_sparse:
        idx[:] = -1
    d = lambda t: None if t is None else t.to(dev)  # noqa: E731
    out = _hip().hip_maba_sa_prefill(d(q), d(k), d(v), d(kh), d(vh), d(early), d(idx), d(gate),
                                     scale=0.125, window=window, n_sink=n_sink, out_dtype=torch.float32)
    exp = osa.maba_sa_prefill_heads(to_np(q), to_np(k), to_np(v), to_np(kh), to_np(vh), to_np(early), idx.numpy(),
                                    to_np(gate), window=window, n_sink=n_sink, scale=0.125)
    assert_close(out, exp, 2e-3, 2e-3, "maba_sa_prefill edge")


def _latent_case(B, H, Lq, Lkv, dc, K, seed, shared=False, gate4=False, dup=False, dh=64):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Lq, dh, generator=g).bfloat16()
    c = torch.randn(B, Lkv, dc, generator=g).bfloat16()
    Wk = (torch.randn(H * dh, dc, generator=g) * dc ** -0.5).bfloat16()
    Wv = (torch.randn(H * dh, dc, generator=g) * dc ** -0.5).bfloat16()
    nb = (Lkv + 63) // 64
    idx = torch.randint(0, nb, (B, 1 if shared else Lq, K), generator=g)
    if K > 2:
        idx[:, :, 0] = -1                                       # an empty slot (ignored)
    if dup and K > 2:
        idx[:, ::3, 2] = idx[:, ::3, 1]                         # repeated blocks count twice
    gate = torch.randn(B, H, Lq, 3, generator=g) if gate4 else torch.randn(B, Lq, 3, generator=g)
    return q, c, Wk, Wv, idx, gate


def _latent_run(dev, q, c, Wk, Wv, idx, gate, window, n_sink, pool=64):
    """The layer's latent composition on the GPU: q_lat = W_k,h^T q_h (fp32), the kernel over the
    bf16 latent rows and their bf16 block means, then W_v,h z."""
    B, H, Lq, dh = q.shape
    dc = c.shape[-1]
    Wk_h = Wk.float().view(H, dh, dc).to(dev)
    Wv_h = Wv.float().view(H, dh, dc).to(dev)
    q_lat = torch.einsum("bhtd,hdc->bthc", q.to(dev).float(), Wk_h).contiguous()
    cd = c.to(dev)
    nc = c.shape[1] // pool
    hca = (_hip().hip_hca_pool(cd[:, : nc * pool], pool=pool) if nc > 0
           else torch.zeros(B, 1, dc, device=dev, dtype=torch.bfloat16))
    z = _hip().hip_maba_sa_prefill_latent(q_lat, cd, hca, idx.to(dev), gate.to(dev), scale=dh ** -0.5,
                                          window=window, n_sink=n_sink, block_size=64, pool=pool)
    return torch.einsum("bthc,hdc->bhtd", z, Wv_h)


@pytest.mark.parametrize("B,H,Lq,Lkv,dc,K,window,n_sink,shared,gate4,dup", [
    (2, 3, 150, 150, 64, 4, 128, 4, False, False, True),    # early rows, two complete means, repeats
    (1, 2, 77, 300, 128, 8, 40, 2, False, True, False),     # a past, per-head gates, narrow window
    (2, 2, 64, 64, 32, 3, 16, 0, True, False, False),       # d_c 32, one index row for all queries
    (1, 2, 40, 40, 128, 2, 128, 4, False, False, False),    # no complete block: all early
    (1, 10, 600, 1000, 128, 32, 128, 4, False, False, True),  # the layer's head count and top-k
    (1, 16, 300, 2000, 96, 16, 300, 70, False, False, False),  # 16 heads, sinks wider than one tile
    (1, 4, 200, 4200, 128, 64, 128, 4, False, True, True),  # 64 index slots
])
def test_maba_sa_prefill_latent_vs_oracle(dev, B, H, Lq, Lkv, dc, K, window, n_sink, shared, gate4, dup):
    q, c, Wk, Wv, idx, gate = _latent_case(B, H, Lq, Lkv, dc, K, B * 1000 + Lq + K, shared, gate4, dup)
    out = _latent_run(dev, q, c, Wk, Wv, idx, gate, window, n_sink)
    exp = osa.maba_sa_prefill(to_np(q), to_np(c), to_np(Wk), to_np(Wv), idx.numpy(), to_np(gate),
                              window=window, n_sink=n_sink)
    assert_close(out, exp, 2e-3, 2e-3, "maba_sa_prefill_latent")


@pytest.mark.parametrize("Lq,Lkv,window,n_sink,empty_sparse", [
    (1, 1, 128, 4, False),      # one token
    (1, 500, 128, 4, False),    # one query over a past: a decode step
    (50, 200, 0, 0, False),     # no local keys at all: the local stream contributes 0
    (40, 100, 16, 200, True),   # sinks wider than the sequence; every index slot empty
    (70, 70, 128, 4, False),    # queries on both sides of the first complete block
])
def test_maba_sa_prefill_latent_edges(dev, Lq, Lkv, window, n_sink, empty_sparse):
    q, c, Wk, Wv, idx, gate = _latent_case(2, 3, Lq, Lkv, 64, 4, Lq * 7 + Lkv)
    if empty_sparse:
        idx[:] = -1
    out = _latent_run(dev, q, c, Wk, Wv, idx, gate, window, n_sink)
    exp = osa.maba_sa_prefill(to_np(q), to_np(c), to_np(Wk), to_np(Wv), idx.numpy(), to_np(gate),
                              window=window, n_sink=n_sink)
    assert_close(out, exp, 2e-3, 2e-3, "maba_sa_prefill_latent edge")


def test_maba_sa_prefill_latent_matches_decode(dev):
    """Every query row of the prefill equals a decode step at that prefix length (the decode
    entry point, with the same index row)."""
    B, H, Lq, Lkv, dc, K = 1, 4, 96, 400, 128, 8
    q, c, Wk, Wv, idx, gate = _latent_case(B, H, Lq, Lkv, dc, K, 5)
    Wk_h = Wk.float().view(H, 64, dc).to(dev)
    q_lat = torch.einsum("bhtd,hdc->bthc", q.to(dev).float(), Wk_h).contiguous()
    cd = c.to(dev)
    hca = _hip().hip_hca_pool(cd, pool=64)
    z = _hip().hip_maba_sa_prefill_latent(q_lat, cd, hca, idx.to(dev), gate.to(dev), scale=0.125)
    for t in (0, 1, 37, Lq - 1):
        L = Lkv - Lq + t + 1
        zd = _hip().hip_maba_sa_decode(q_lat[:, t].contiguous(), cd, hca, idx[:, t: t + 1].to(dev),
                                       gate[:, t].to(dev), L=L, scale=0.125)
        err = (z[:, t] - zd).abs().max().item()
        assert err <= 1e-4 * max(1.0, zd.abs().max().item()), (t, err)
