"""HIP kernels vs the CPU oracle on seeded inputs (runs on the GPU box).

Tolerances: fp32 paths 1e-4 (reference test_cpu_dgda.py:469-470,
test_triton_indexer.py:124-145); mixed bf16-input / fp32-accumulate paths
rtol = atol = 2e-3; block indices bit-exact wherever the
oracle's scores separate them by more than 1e-4.
"""
import math

import numpy as np
import pytest
import torch

from _helpers import assert_close, dgda_inputs, oracle_dgda_args, to_np, topk_agrees, topk_is_valid
from oracle import dgda as odgda
from oracle import indexer as oidx
from oracle import sparse_attn as osa

pytestmark = pytest.mark.gpu


def _hip():
    from maba_sparse.kernels import hip_backend
    return hip_backend


# ----------------------------------------------------------------------------- dgda_step

@pytest.mark.parametrize("B,H,dk,dv", [(2, 3, 64, 64), (64, 10, 64, 64), (3, 2, 32, 128), (1, 1, 128, 16), (2, 2, 17, 33)])
def test_dgda_step_fp32(dev, B, H, dk, dv):
    g = torch.Generator().manual_seed(B * 100 + dk)
    q = torch.randn(B, H, dk, generator=g)
    k = torch.nn.functional.normalize(torch.randn(B, H, dk, generator=g), dim=-1)
    v = torch.randn(B, H, dv, generator=g)
    la = -torch.nn.functional.softplus(torch.randn(B, H, dk, generator=g) + 2)
    b = torch.sigmoid(torch.randn(B, H, dk, generator=g))
    w = torch.sigmoid(torch.randn(B, H, dv, generator=g))
    S = torch.randn(B, H, dk, dv, generator=g)
    o, Sn = _hip().hip_dgda_step(q.to(dev), k.to(dev), v.to(dev), log_alpha=la.to(dev), b=b.to(dev),
                                 w=w.to(dev), state=S.to(dev))
    eo, eS = odgda.dgda_step(q, k, v, alpha=np.exp(to_np(la)), b=b, w=w, state=to_np(S))
    assert_close(o, eo, 1e-4, 1e-4, "out")
    assert_close(Sn, eS, 1e-4, 1e-4, "state")


@pytest.mark.parametrize("dk", [32, 64, 128])
@pytest.mark.parametrize("dv", [32, 64, 128])
@pytest.mark.parametrize("sdt", [torch.float32, torch.bfloat16])
def test_dgda_step_head_sizes_fast_kernel(dev, dk, dv, sdt):
    """The four-wave step kernel at every head size of the reference's GPU path (d_k, d_v in
    {32, 64, 128}, contiguous state rows): bf16 q/k/v, fp32 gates, fp32 or bf16 state updated in
    place, against the float64 step on the same (rounded) inputs; and with no state."""
    B, H = 6, 3
    g = torch.Generator().manual_seed(dk * 7 + dv)
    q = torch.randn(B, H, dk, generator=g).bfloat16()
    k = torch.nn.functional.normalize(torch.randn(B, H, dk, generator=g), dim=-1).bfloat16()
    v = torch.randn(B, H, dv, generator=g).bfloat16()
    la = -torch.nn.functional.softplus(torch.randn(B, H, dk, generator=g) + 2)
    b = torch.sigmoid(torch.randn(B, H, dk, generator=g))
    w = torch.sigmoid(torch.randn(B, H, dv, generator=g))
    S0 = (torch.randn(B, H, dk, dv, generator=g) * 0.5).to(sdt)
    S = S0.to(dev)
    o, Sn = _hip().hip_dgda_step(q.to(dev), k.to(dev), v.to(dev), log_alpha=la.to(dev), b=b.to(dev), w=w.to(dev),
                                 state=S, new_state=S, out_dtype=torch.float32, state_dtype=sdt,
                                 allow_mixed_dtypes=True)
    assert Sn.data_ptr() == S.data_ptr()
    eo, eS = odgda.dgda_step(to_np(q), to_np(k), to_np(v), alpha=np.exp(to_np(la)), b=to_np(b), w=to_np(w),
                             state=to_np(S0))
    tol = 1e-4 if sdt == torch.float32 else 8e-3    # bf16 state: the stored state is rounded to bf16
    assert_close(o, eo, tol, tol, f"out dk={dk} dv={dv}")
    assert_close(Sn, eS, tol, tol, f"state dk={dk} dv={dv}")
    o0, S1 = _hip().hip_dgda_step(q.to(dev), k.to(dev), v.to(dev), log_alpha=la.to(dev), b=b.to(dev), w=w.to(dev),
                                  out_dtype=torch.float32, state_dtype=torch.float32, allow_mixed_dtypes=True)
    eo0, eS1 = odgda.dgda_step(to_np(q), to_np(k), to_np(v), alpha=np.exp(to_np(la)), b=to_np(b), w=to_np(w))
    assert_close(o0, eo0, 1e-4, 1e-4, "out, no state")
    assert_close(S1, eS1, 1e-4, 1e-4, "state, no state")


def test_dgda_step_4d_alpha_no_state(dev):
    g = torch.Generator().manual_seed(7)
    B, H, d = 4, 2, 64
    q, k, v = (torch.randn(B, H, 1, d, generator=g) for _ in range(3))
    a = torch.rand(B, H, 1, d, generator=g)
    b, w = torch.rand(B, H, 1, d, generator=g), torch.rand(B, H, 1, d, generator=g)
    o, Sn = _hip().hip_dgda_step(*(t.to(dev) for t in (q, k, v)), alpha=a.to(dev), b=b.to(dev), w=w.to(dev))
    eo, eS = odgda.dgda_step(q, k, v, alpha=a, b=b, w=w)
    assert o.shape == (B, H, d)
    assert_close(o, eo, 1e-4, 1e-4, "out")
    assert_close(Sn, eS, 1e-4, 1e-4, "state")


def test_dgda_step_mixed_bf16(dev):
    """BASELINE decode microbench dtypes: bf16 q/k/v, fp32 gates and state."""
    inp = dgda_inputs(64, 10, 1, seed=3, device=dev, with_state=True)
    sq = lambda t: t[:, :, 0]
    o, Sn = _hip().hip_dgda_step(sq(inp["q"]), sq(inp["k"]), sq(inp["v"]), log_alpha=sq(inp["log_alpha"]),
                                 b=sq(inp["b"]), w=sq(inp["w"]), state=inp["initial_state"],
                                 out_dtype=torch.float32, state_dtype=torch.float32, allow_mixed_dtypes=True)
    ar = oracle_dgda_args(inp)
    eo, eS = odgda.dgda_step(ar["q"][:, :, 0], ar["k"][:, :, 0], ar["v"][:, :, 0], alpha=ar["alpha"][:, :, 0],
                             b=ar["b"][:, :, 0], w=ar["w"][:, :, 0], state=ar["initial_state"])
    assert_close(o, eo, 2e-3, 2e-3, "out")
    assert_close(Sn, eS, 2e-3, 2e-3, "state")


# ----------------------------------------------------------------------------- dgda_prefill (general path)

@pytest.mark.parametrize("gates", ["channel", "scalar"])
@pytest.mark.parametrize("L", [1, 17, 200])
def test_dgda_prefill_fp32(dev, gates, L):
    inp = dgda_inputs(2, 3, L, 64, 64, qkv_dtype=torch.float32, gates=gates, seed=L, device=dev, with_state=True)
    o, S = _hip().hip_dgda_prefill(**inp)
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 1e-4, 1e-4, "out")
    assert_close(S, eS, 1e-4, 1e-4, "state")


def test_dgda_prefill_odd_dims(dev):
    inp = dgda_inputs(1, 2, 33, 24, 40, qkv_dtype=torch.float32, gates="channel", seed=5, device=dev)
    o, S = _hip().hip_dgda_prefill(**inp)
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 1e-4, 1e-4, "out")
    assert_close(S, eS, 1e-4, 1e-4, "state")


def test_dgda_prefill_transposed_views(dev):
    """The layer passes [B,L,H,d] storage viewed as [B,H,L,d] (dgda.py:199-205)."""
    B, L, H, d = 2, 40, 3, 64
    g = torch.Generator().manual_seed(11)
    phys = [torch.randn(B, L, H, d, generator=g) for _ in range(3)]
    q, k, v = (p.to(dev).transpose(1, 2) for p in phys)
    k = k / k.norm(dim=-1, keepdim=True)
    la = (-torch.nn.functional.softplus(torch.randn(B, L, H, d, generator=g))).to(dev).transpose(1, 2)
    b = torch.rand(B, L, H, d, generator=g).to(dev).transpose(1, 2)
    w = torch.rand(B, L, H, d, generator=g).to(dev).transpose(1, 2)
    o, S = _hip().hip_dgda_prefill(q, k, v, log_alpha=la, b=b, w=w)
    eo, eS = odgda.dgda_prefill_seq(to_np(q), to_np(k), to_np(v), alpha=np.exp(to_np(la)), b=to_np(b), w=to_np(w))
    assert_close(o, eo, 1e-4, 1e-4, "out")
    assert_close(S, eS, 1e-4, 1e-4, "state")


# ----------------------------------------------------------------------------- pooling

@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 1e-2), (torch.float16, 5e-3)])
@pytest.mark.parametrize("B,L,d", [(1, 64, 64), (2, 100, 64), (3, 1, 128), (2, 4096, 128), (1, 70, 96), (2, 65, 30)])
def test_compute_centroids(dev, dtype, tol, B, L, d):
    x = torch.randn(B, L, d, generator=torch.Generator().manual_seed(L + d)).to(dtype)
    c = _hip().hip_compute_centroids(x.to(dev), block_size=64)
    exp = oidx.compute_centroids(to_np(x), 64)
    assert c.dtype == dtype
    assert_close(c, exp, 0, tol, "centroids")


def test_compute_centroids_known_answers(dev):
    k = torch.full((1, 256, 64), 0.01, device=dev)
    k[0, 70, :] = 10.0
    c = _hip().hip_compute_centroids(k, block_size=64)
    pure_mean = (63 * 0.01 + 10.0) / 64.0
    assert abs(c[0, 1, 0].item() - 0.5 * (pure_mean + 10.0)) < 1e-3       # test_triton_indexer.py:147-158
    k = torch.full((1, 100, 64), -2.0, device=dev)
    c = _hip().hip_compute_centroids(k, block_size=64)
    assert torch.allclose(c[0, 0], torch.tensor(-2.0, device=dev), atol=1e-4)
    assert torch.allclose(c[0, 1], torch.tensor(0.5 * (-72.0 / 64.0), device=dev), atol=1e-4)  # :160-168


def test_hca_pool(dev):
    x = torch.randn(3, 64 * 7 + 13, 128, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    m = _hip().hip_hca_pool(x.to(dev), pool=64)
    exp = osa.hca_means(to_np(x), pool=64)
    assert m.shape == (3, 7, 128)
    assert_close(m, exp, 0, 1e-2, "hca means")


# ----------------------------------------------------------------------------- superposition

@pytest.mark.parametrize("gate_dim", [3, 4])
@pytest.mark.parametrize("weights", [False, True])
def test_stream_superposition(dev, gate_dim, weights):
    B, H, L, D = 2, 4, 15, 64
    g = torch.Generator().manual_seed(gate_dim + 10 * weights)
    ol, os_, oh = (torch.randn(B, H, L, D, generator=g) for _ in range(3))
    z = torch.randn(*((B, L, 3) if gate_dim == 3 else (B, H, L, 3)), generator=g)
    gate = torch.softmax(z, -1) if weights else z
    kw = {"gate_weights": gate.to(dev)} if weights else {"gate_logits": gate.to(dev)}
    out = _hip().hip_stream_superposition(ol.to(dev), os_.to(dev), oh.to(dev), **kw)
    exp = osa.superposition(to_np(ol), to_np(os_), to_np(oh), **({"gate_weights": to_np(gate)} if weights
                                                                 else {"gate_logits": to_np(gate)}))
    assert_close(out, exp, 1e-5, 1e-5, "superposition")


@pytest.mark.parametrize("case", ["bf16_vec", "bf16_odd_d", "strided_f32", "f16_generic", "bf16_4d_gate"])
def test_stream_superposition_layouts(dev, case):
    """The 16-byte vector kernel (contiguous bf16 / fp32, D a multiple of the vector) and
    the generic one (strided views, other D, fp16) against the fp64 oracle."""
    g = torch.Generator().manual_seed(len(case))
    B, H, L, D = 2, 3, 37, (6 if case == "bf16_odd_d" else 64)
    dt = {"strided_f32": torch.float32, "f16_generic": torch.float16}.get(case, torch.bfloat16)
    ol, os_, oh = (torch.randn(B, H, L, D, generator=g).to(dt) for _ in range(3))
    z = torch.randn(*((B, H, L, 3) if case == "bf16_4d_gate" else (B, L, 3)), generator=g)
    args = [x.to(dev) for x in (ol, os_, oh)]
    if case == "strided_f32":   # [B, L, H, D] storage seen as [B, H, L, D]
        args = [x.transpose(1, 2).contiguous().transpose(1, 2) for x in args]
    out = _hip().hip_stream_superposition(*args, gate_logits=z.to(dev))
    exp = osa.superposition(to_np(ol.float()), to_np(os_.float()), to_np(oh.float()), gate_logits=to_np(z))
    tol = 1e-5 if dt == torch.float32 else 1e-2
    assert out.dtype == dt
    assert_close(out.float(), exp, tol, tol, f"superposition {case}")


def test_superposition_partition_of_unity(dev):
    x = torch.randn(2, 4, 64, 64, device=dev)
    out = _hip().hip_stream_superposition(x, x, x, gate_logits=torch.randn(2, 64, 3, device=dev))
    assert torch.allclose(out, x, atol=1e-5)


# ----------------------------------------------------------------------------- indexer

@pytest.mark.parametrize("B,Hq,nb,d,k,lam,dtype", [
    (2, 10, 15625 // 25, 128, 32, 0.1, torch.bfloat16),
    (1, 1, 8, 64, 32, 0.5, torch.float32),
    (3, 4, 300, 64, 8, 1.0, torch.float32),
    (2, 16, 1000, 128, 64, 0.1, torch.bfloat16),
    (1, 2, 64, 32, 1, 0.0, torch.float16),
])
def test_index_topk_decode(dev, B, Hq, nb, d, k, lam, dtype):
    g = torch.Generator().manual_seed(nb + d)
    q = torch.randn(B, Hq, d, generator=g).to(dtype)
    c = torch.randn(B, nb, d, generator=g).to(dtype)
    idx, sc = _hip().hip_index_topk_decode(q.to(dev), c.to(dev), lambda_dist=lam, top_k=k, return_scores=True)
    ref = oidx.decode_scores(to_np(q), to_np(c), lam)
    assert idx.shape == (B, Hq, min(k, nb)) and idx.dtype == torch.long
    assert_close(sc, ref, 1e-5, 1e-4, "decode scores")
    n = topk_agrees(idx.cpu().numpy(), ref, k)
    assert n >= 1


@pytest.mark.parametrize("nb,lam", [(100, 0.0), (4000, 0.0), (15625, 0.0), (4000, 0.1)])
def test_index_topk_decode_ties(dev, nb, lam):
    """Zero centroids: every score is the penalty alone.  With lam = 0 all scores tie and
    the order is index ascending (nb = 4000 and 15625 exceed the select kernel's
    candidate slots and take the merge fallback); with lam > 0 the penalty decreases
    toward the last block, so the picks are the last blocks, newest first."""
    q = torch.randn(2, 10, 128, generator=torch.Generator().manual_seed(5)).to(dev, torch.bfloat16)
    c = torch.zeros(2, nb, 128, device=dev, dtype=torch.bfloat16)
    idx = _hip().hip_index_topk_decode(q, c, lambda_dist=lam, top_k=32)
    exp = torch.arange(32) if lam == 0.0 else torch.arange(nb - 1, nb - 33, -1)
    assert torch.equal(idx.cpu(), exp.expand(2, 10, 32))


def test_index_topk_decode_near_equal_centroids(dev):
    """The DGDA layer's situation: centroids 0.5 (mean + max) of random keys are nearly
    equal, so the distance penalty orders most of the row and the group-maximum bound
    admits thousands of candidates (the merge fallback).  One query head, d = 64."""
    g = torch.Generator().manual_seed(21)
    B, Hq, nb, d = 4, 1, 15625, 64
    keys = torch.randn(B, nb * 64 // 16, d, generator=g)        # a quarter-size key sample per block
    c = (0.5 * (keys.view(B, nb, 4, d).mean(2) + keys.view(B, nb, 4, d).amax(2))).bfloat16()
    q = torch.randn(B, Hq, d, generator=g).bfloat16()
    idx, sc = _hip().hip_index_topk_decode(q.to(dev), c.to(dev), lambda_dist=0.1, top_k=32, return_scores=True)
    ref = oidx.decode_scores(to_np(q), to_np(c), 0.1)
    assert_close(sc, ref, 1e-5, 1e-4, "decode scores")
    assert topk_agrees(idx.cpu().numpy(), ref, 32) >= B * Hq - 1


def test_index_topk_decode_tied_plateau(dev):
    """300 planted blocks share the top score (positive queries, identical centroids),
    every other centroid is zero and lam = 0: the top 32 are the 32 lowest planted
    indices.  The tied plateau spreads over the whole row, so the select kernel ranks a
    few hundred candidates by counting (neither the register rank nor the merge fallback)."""
    g = torch.Generator().manual_seed(12)
    B, Hq, nb, d = 2, 10, 15625, 128
    q = torch.randn(B, Hq, d, generator=g).abs().bfloat16()
    c = torch.zeros(B, nb, d, dtype=torch.bfloat16)
    exp = []
    for b in range(B):
        blocks = torch.randperm(nb, generator=g)[:300]
        c[b, blocks] = 0.5
        exp.append(torch.sort(blocks).values[:32])
    idx = _hip().hip_index_topk_decode(q.to(dev), c.to(dev), lambda_dist=0.0, top_k=32)
    assert torch.equal(idx.cpu(), torch.stack(exp)[:, None, :].expand(B, Hq, 32))


def test_index_topk_decode_baseline_needle(dev):
    """BASELINE config 3 shape for one batch element pair: 15,625 bf16 centroids with a
    planted block; the needle block is selected first for every head aligned with it and
    the full top-32 matches the oracle wherever its scores separate."""
    g = torch.Generator().manual_seed(11)
    B, Hq, nb, d = 2, 10, 15625, 128
    c = torch.randn(B, nb, d, generator=g).bfloat16()
    q = torch.randn(B, Hq, d, generator=g).bfloat16()
    c[0, 777] = (q[0, 3].float() * 4).bfloat16()          # needle aligned with head 3
    idx, sc = _hip().hip_index_topk_decode(q.to(dev), c.to(dev), lambda_dist=0.1, top_k=32, return_scores=True)
    ref = oidx.decode_scores(to_np(q), to_np(c), 0.1)
    assert_close(sc, ref, 1e-5, 1e-4, "decode scores")
    assert idx[0, 3, 0].item() == 777
    assert topk_agrees(idx.cpu().numpy(), ref, 32) >= B * Hq - 2


@pytest.mark.parametrize("B,L,nb_blocks,k,lam", [(1, 64, 1, 1, 0.5), (2, 128, 2, 2, 0.5), (3, 256, 4, 4, 0.5),
                                                  (2, 512, 8, 8, 1.0), (1, 100, 2, 2, 0.25), (2, 65, 2, 2, 0.0),
                                                  (2, 16, 1, 2, 0.5), (1, 512, 8, 32, 0.5), (2, 4096, 64, 32, 0.1)])
def test_index_topk_prefill(dev, B, L, nb_blocks, k, lam):
    g = torch.Generator().manual_seed(L + k)
    q = torch.randn(B, L, 64, generator=g)
    kk = torch.randn(B, L, 64, generator=g)
    cent = torch.from_numpy(oidx.compute_centroids(to_np(kk), 64)).float()
    idx, sc = _hip().hip_index_topk(q.to(dev), cent.to(dev), lambda_dist=lam, top_k=k, block_size=64,
                                    return_scores=True)
    ref = oidx.prefill_scores(to_np(q), to_np(cent), lam, 64)
    fin = np.isfinite(ref)
    assert_close(sc.cpu().numpy()[fin], ref[fin], 1e-5, 1e-4, "scores")
    assert np.all(np.isneginf(sc.cpu().numpy()[~fin]))
    topk_agrees(idx.cpu().numpy(), ref, k)
    # causal: the first min(k, qblk+1) picks are past or current blocks
    ii = idx.cpu().numpy()
    for t in range(L):
        avail = min(t // 64 + 1, ii.shape[-1])
        assert (ii[:, t, :avail] <= t // 64).all()


@pytest.mark.parametrize("B,L,nb,d,k,lam,bs", [(2, 1000, 16, 128, 8, 0.5, 64), (1, 4096, 64, 64, 32, 0.1, 64),
                                                (3, 333, 11, 96, 4, 1.0, 32), (1, 50, 1, 32, 8, 0.5, 64),
                                                (2, 700, 24, 128, 32, 0.0, 32)])
def test_index_topk_prefill_bf16_mfma(dev, B, L, nb, d, k, lam, bs):
    """bf16 queries and centroids without score output take the MFMA prefill kernel
    (16 query rows per workgroup): picks agree with the float64 oracle wherever its
    scores separate, equal the fp32 kernel's on the same values, and rows that see
    fewer blocks than k end with the masked blocks in index order."""
    g = torch.Generator().manual_seed(L + d)
    q = torch.randn(B, L, d, generator=g).bfloat16()
    cent = torch.randn(B, nb, d, generator=g).bfloat16()
    idx = _hip().hip_index_topk(q.to(dev), cent.to(dev), lambda_dist=lam, top_k=k, block_size=bs)
    ak = min(k, nb)
    assert idx.shape == (B, L, ak) and idx.dtype == torch.long
    ref = oidx.prefill_scores(to_np(q), to_np(cent), lam, bs)
    assert topk_agrees(idx.cpu().numpy(), ref, k) > 0
    ii = idx.cpu().numpy()
    for t in range(L):
        avail = min(t // bs + 1, nb)
        if avail < ak:
            assert (np.sort(ii[:, t, :avail], axis=-1) == np.arange(avail)).all()
            assert (ii[:, t, avail:] == np.arange(avail, ak)).all()
    idx32, _ = _hip().hip_index_topk(q.float().to(dev), cent.float().to(dev), lambda_dist=lam, top_k=k, block_size=bs,
                                     return_scores=True)
    same = (idx32.cpu().numpy() == ii).all(axis=-1).mean()
    assert same > 0.99, same


def test_index_topk_penalty_order(dev):
    q = torch.ones(1, 256, 64, device=dev) / 8.0
    c = torch.ones(1, 4, 64, device=dev) / 8.0
    idx = _hip().hip_index_topk(q, c, lambda_dist=1.0, top_k=4, block_size=64)
    assert idx[0, 255].tolist() == [3, 2, 1, 0]      # test_triton_indexer.py:247-255


# ----------------------------------------------------------------------------- MABA-SA decode

def _sa_case(B, H, dh, dc, L, K, Hi, seed, dev, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    c = torch.randn(B, L, dc, generator=g).to(dtype)
    Wk = (torch.randn(H * dh, dc, generator=g) * 0.05)
    Wv = (torch.randn(H * dh, dc, generator=g) * 0.05)
    q = torch.randn(B, H, dh, generator=g)
    nb = (L + 63) // 64
    idx = torch.stack([torch.stack([torch.randperm(nb, generator=g)[: min(K, nb)] for _ in range(Hi)])
                       for _ in range(B)])
    gate = torch.randn(B, 3, generator=g)
    return c, Wk, Wv, q, idx, gate


@pytest.mark.parametrize("L,K,Hi", [(1, 32, 1), (50, 32, 1), (64, 32, 1), (200, 32, 1), (1000, 8, 1),
                                    (3000, 32, 4), (5000, 32, 1)])
def test_maba_sa_decode(dev, L, K, Hi):
    B, H, dh, dc = 2, 4, 64, 128
    c, Wk, Wv, q, idx, gate = _sa_case(B, H, dh, dc, L, K, Hi, L + K, dev)
    hca = _hip().hip_hca_pool(c.to(dev), pool=64)
    Wk_h = Wk.view(H, dh, dc)
    q_lat = torch.einsum("bhd,hdc->bhc", q, Wk_h)          # W_k,h^T q_h
    z = _hip().hip_maba_sa_decode(q_lat.to(dev), c.to(dev), hca, idx.to(dev), gate.to(dev), L=L,
                                  scale=1.0 / math.sqrt(dh))
    out = torch.einsum("bhc,hdc->bhd", z.cpu(), Wv.view(H, dh, dc))
    exp = osa.maba_sa_decode(to_np(q), to_np(c), to_np(Wk), to_np(Wv), to_np(idx).astype(np.int64),
                             to_np(gate), means=to_np(hca))
    assert_close(out, exp, 2e-3, 2e-3, "maba_sa")


@pytest.mark.parametrize("L,window,n_sink", [(5000, 1000, 4), (3000, 2999, 0), (700, 650, 16)])
def test_maba_sa_decode_wide_window(dev, L, window, n_sink):
    """Windows of many 64-key tiles: the local stream is cut into several segments."""
    B, H, dh, dc, K = 2, 4, 64, 128, 16
    c, Wk, Wv, q, idx, gate = _sa_case(B, H, dh, dc, L, K, 1, L + window, dev)
    hca = _hip().hip_hca_pool(c.to(dev), pool=64)
    q_lat = torch.einsum("bhd,hdc->bhc", q, Wk.view(H, dh, dc))
    z = _hip().hip_maba_sa_decode(q_lat.to(dev), c.to(dev), hca, idx.to(dev), gate.to(dev), L=L,
                                  scale=1.0 / math.sqrt(dh), window=window, n_sink=n_sink)
    out = torch.einsum("bhc,hdc->bhd", z.cpu(), Wv.view(H, dh, dc))
    exp = osa.maba_sa_decode(to_np(q), to_np(c), to_np(Wk), to_np(Wv), to_np(idx).astype(np.int64),
                             to_np(gate), window=window, n_sink=n_sink, means=to_np(hca))
    assert_close(out, exp, 2e-3, 2e-3, "maba_sa wide window")


@pytest.mark.parametrize("L,K,Hi", [(8192, 64, 10), (20000, 64, 1)])
def test_maba_sa_decode_many_segments(dev, L, K, Hi):
    """Enough tiles that every wave runs several tiles (register prefetch path) and the
    combine merges partials from many workgroups."""
    B, H, dh, dc = 4, 10, 64, 128
    c, Wk, Wv, q, idx, gate = _sa_case(B, H, dh, dc, L, K, Hi, L + K + 1, dev)
    hca = _hip().hip_hca_pool(c.to(dev), pool=64)
    q_lat = torch.einsum("bhd,hdc->bhc", q, Wk.view(H, dh, dc))
    z = _hip().hip_maba_sa_decode(q_lat.to(dev), c.to(dev), hca, idx.to(dev), gate.to(dev), L=L,
                                  scale=1.0 / math.sqrt(dh))
    out = torch.einsum("bhc,hdc->bhd", z.cpu(), Wv.view(H, dh, dc))
    exp = osa.maba_sa_decode(to_np(q), to_np(c), to_np(Wk), to_np(Wv), to_np(idx).astype(np.int64),
                             to_np(gate), means=to_np(hca))
    assert_close(out, exp, 2e-3, 2e-3, "maba_sa")


# ----------------------------------------------------------------------------- top_k > 64
# The reference takes any K (common.py:353-403, cpu_indexer.py:53-112, layers/indexer.py:101-112);
# past the 64-key wave lists the general path scores each row and sorts it in LDS.

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("nb,k", [(300, 65), (1000, 128), (15625, 256), (200, 200)])
def test_index_topk_decode_large_k(dev, nb, k, dtype):
    g = torch.Generator().manual_seed(nb + k)
    B, Hq, d = 2, 3, 128
    q = torch.randn(B, Hq, d, generator=g).to(dtype)
    c = torch.randn(B, nb, d, generator=g).to(dtype)
    idx, sc = _hip().hip_index_topk_decode(q.to(dev), c.to(dev), lambda_dist=0.1, top_k=k, return_scores=True)
    ref = oidx.decode_scores(to_np(q), to_np(c), 0.1)
    assert idx.shape == (B, Hq, min(k, nb))
    assert_close(sc, ref, 1e-5, 1e-4, "decode scores")
    assert topk_agrees(idx.cpu().numpy(), ref, k) >= B * Hq - 1
    topk_is_valid(idx.cpu().numpy(), ref)


@pytest.mark.parametrize("L,k,lam", [(9000, 100, 0.5), (12800, 200, 0.1), (5000, 79, 0.0)])
def test_index_topk_prefill_large_k(dev, L, k, lam):
    """Causal prefill with K > 64: rows with fewer live blocks than K fill the remaining slots
    with the lowest masked blocks; the returned scores are the oracle's (-inf where masked)."""
    g = torch.Generator().manual_seed(L + k)
    B, d = 2, 64
    q = torch.randn(B, L, d, generator=g)
    keys = torch.randn(B, L, d, generator=g)
    cent = torch.from_numpy(oidx.compute_centroids(to_np(keys), 64)).float()
    nb = cent.shape[1]
    idx, sc = _hip().hip_index_topk(q.to(dev), cent.to(dev), lambda_dist=lam, top_k=k, block_size=64,
                                    return_scores=True)
    ref = oidx.prefill_scores(to_np(q), to_np(cent), lam)
    ak = min(k, nb)
    assert idx.shape == (B, L, ak)
    got_sc = sc.double().cpu().numpy()
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(got_sc), fin)
    assert np.allclose(got_sc[fin], ref[fin], rtol=1e-5, atol=1e-4)
    got = idx.cpu().numpy()
    rows = [0, 63, 64, 1000, L // 2, L - 1]
    sub = got[:, rows]
    assert topk_agrees(sub, ref[:, rows], k) >= 1
    topk_is_valid(sub, np.where(fin[:, rows], ref[:, rows], -1e30))
    for t in rows:                                # masked slots: the lowest masked blocks, ascending
        live = min(t // 64 + 1, nb)
        if live < ak:
            assert (got[:, t, live:] == np.arange(live, ak)).all()
