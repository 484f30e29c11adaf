"""Every op-level entry point captured in a HIP graph and replayed: the library's kernels
take their stream from the caller and allocate nothing, so a captured call must replay to
the eager call's results.  Each case runs the op eagerly, captures it (after a warm-up on a
side stream), then replays the graph three times with eager work of the same op and a
synchronisation between the replays, and requires every replay's outputs to equal the
eager outputs bit for bit (the same kernels on the same inputs).

Covered: the chunked DGDA prefill (three launches), the sub-chunk prefill at d_v = 128 (two
calls of three launches over the value halves), the fused layer prefill, the decode step,
both decode top-k paths (K <= 64 and the sorted path above 64), the MABA-SA decode
(segments + merge), both MABA-SA prefill kernels and the block pooling; and two streams
calling the library at the same time.
"""
import pytest
import torch

from _helpers import dgda_inputs

pytestmark = pytest.mark.gpu


def _hip():
    from maba_sparse.kernels import hip_backend
    return hip_backend


def _as_tuple(x):
    return tuple(t for t in (x if isinstance(x, (tuple, list)) else (x,)) if isinstance(t, torch.Tensor))


def _check_replays(fn, replays=3):
    eager = [t.clone() for t in _as_tuple(fn())]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = _as_tuple(fn())
    assert len(captured) == len(eager)
    for r in range(replays):
        fn()                              # eager work of the same op between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, want) in enumerate(zip(captured, eager)):
            assert torch.equal(got, want), f"replay {r}, output {i} differs from the eager call"


def test_graph_dgda_prefill_chunked(dev):
    inp = dgda_inputs(1, 2, 4096, seed=1, device=dev)          # per-token gates: the chunked path
    _check_replays(lambda: _hip().hip_dgda_prefill(**inp, out_dtype=torch.bfloat16, state_dtype=torch.float32,
                                                   allow_mixed_dtypes=True))


def test_graph_dgda_prefill_subchunk_dv128(dev):
    inp = dgda_inputs(1, 2, 2100, dk=64, dv=128, seed=2, decay="slow", gates="channel", device=dev,
                      with_state=True)
    _check_replays(lambda: _hip().hip_dgda_prefill(**inp, out_dtype=torch.float32, state_dtype=torch.float32,
                                                   allow_mixed_dtypes=True))


def test_graph_dgda_layer_prefill(dev):
    B, T, H = 2, 1500, 3
    C = 64 * H
    g = torch.Generator(device=dev).manual_seed(3)
    projs = [torch.randn(B, T, C, device=dev, generator=g, dtype=torch.bfloat16) for _ in range(6)]
    ws = [torch.randn(C, 1, 4, device=dev, generator=g) * 0.3 for _ in range(3)]
    hist = [torch.randn(B, C, 3, device=dev, generator=g, dtype=torch.bfloat16) for _ in range(3)]
    _check_replays(lambda: _hip().hip_dgda_layer_prefill(projs, ws, hist, state_dtype=torch.float32))


def test_graph_dgda_step(dev):
    B, H, d = 16, 4, 128
    g = torch.Generator(device=dev).manual_seed(4)
    q, k, v = (torch.randn(B, H, d, device=dev, generator=g).bfloat16() for _ in range(3))
    la = -torch.rand(B, H, d, device=dev, generator=g)
    b, w = torch.rand(B, H, d, device=dev, generator=g), torch.rand(B, H, d, device=dev, generator=g)
    S = torch.randn(B, H, d, d, device=dev, generator=g) * 0.1
    _check_replays(lambda: _hip().hip_dgda_step(q, k, v, b=b, w=w, state=S, log_alpha=la, out_dtype=torch.float32,
                                                state_dtype=torch.float32, allow_mixed_dtypes=True))


@pytest.mark.parametrize("K", [32, 100])
def test_graph_index_topk_decode(dev, K):
    g = torch.Generator(device=dev).manual_seed(5)
    q = torch.randn(4, 8, 128, device=dev, generator=g).bfloat16()
    cent = torch.randn(4, 3000, 128, device=dev, generator=g).bfloat16()
    _check_replays(lambda: _hip().hip_index_topk_decode(q, cent, lambda_dist=0.1, top_k=K, return_scores=True))


def test_graph_maba_sa_decode_and_pooling(dev):
    B, H, dc, L, K = 4, 10, 128, 20000, 32
    g = torch.Generator(device=dev).manual_seed(6)
    c = torch.randn(B, L, dc, device=dev, generator=g).bfloat16()
    q_lat = torch.randn(B, H, dc, device=dev, generator=g)
    nb = (L + 63) // 64
    idx = torch.randint(0, nb, (B, H, K), device=dev, generator=g)
    gate = torch.randn(B, H, 3, device=dev, generator=g)
    hca = _hip().hip_hca_pool(c, pool=64)
    _check_replays(lambda: _hip().hip_hca_pool(c, pool=64))
    _check_replays(lambda: _hip().hip_compute_centroids(c, block_size=64))
    _check_replays(lambda: _hip().hip_maba_sa_decode(q_lat, c, hca, idx, gate, L=L, scale=0.125))


def test_graph_maba_sa_prefill_both_kernels(dev):
    B, H, L, dh, dc, K = 1, 4, 2100, 64, 128, 16
    g = torch.Generator(device=dev).manual_seed(7)
    bf = lambda *sh: torch.randn(*sh, device=dev, generator=g, dtype=torch.bfloat16)  # noqa: E731
    q, k, v = bf(B, H, L, dh), bf(B, H, L, dh), bf(B, H, L, dh)
    kh, vh = bf(B, H, L // 64, dh), bf(B, H, L // 64, dh)
    early = bf(B, H, 63, dh)
    c = bf(B, L, dc)
    q_lat = torch.randn(B, L, H, dc, device=dev, generator=g)
    pos_blk = torch.arange(L, device=dev) // 64
    idx = (torch.rand(B, L, K, device=dev, generator=g) * (pos_blk[None, :, None] + 1).float()).long()
    gate = torch.randn(B, L, 3, device=dev, generator=g)
    hca = _hip().hip_hca_pool(c, pool=64)
    _check_replays(lambda: _hip().hip_maba_sa_prefill(q, k, v, kh, vh, early, idx, gate, scale=0.125))
    _check_replays(lambda: _hip().hip_maba_sa_prefill_latent(q_lat, c, hca, idx, gate, scale=0.125))


def test_two_streams_at_once(dev):
    """Calls on two streams at the same time (each with its own workspace) give the results of
    the same calls one after the other: the library keeps no per-call state between calls."""
    hb = _hip()
    inp = dgda_inputs(2, 3, 3000, seed=8, gates="channel", device=dev)
    g = torch.Generator(device=dev).manual_seed(9)
    q = torch.randn(4, 8, 128, device=dev, generator=g).bfloat16()
    cent = torch.randn(4, 5000, 128, device=dev, generator=g).bfloat16()
    pre = lambda: hb.hip_dgda_prefill(**inp, out_dtype=torch.float32, state_dtype=torch.float32,  # noqa: E731
                                      allow_mixed_dtypes=True)
    top = lambda: hb.hip_index_topk_decode(q, cent, lambda_dist=0.1, top_k=32, return_scores=True)  # noqa: E731
    want_pre = [t.clone() for t in pre()]
    want_top = [t.clone() for t in top()]
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    for _ in range(3):
        sa.wait_stream(torch.cuda.current_stream())
        sb.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(sa):
            got_pre = pre()
        with torch.cuda.stream(sb):
            got_top = top()
        torch.cuda.synchronize()
        for a, b in zip(got_pre, want_pre):
            assert torch.equal(a, b)
        for a, b in zip(got_top, want_top):
            assert torch.equal(a, b)
