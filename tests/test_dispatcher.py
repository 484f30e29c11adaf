"""Host-side dispatcher contract (reference: maba_sparse/kernels/dispatcher.py and
tests/test_dispatcher_fallbacks.py), on the CPU.

Routing and the ``MABA_BACKEND`` override, the registry API, the once-per-op
fallback warning and its strict-mode escalation, propagation of a missing HIP
library, and the HIP wrappers' refusal of autograd and of CPU tensors.
"""
import threading
import warnings

import pytest
import torch

from maba_sparse._native import HipLibraryMissing
from maba_sparse.kernels import dispatcher as D
from maba_sparse.kernels import common as C


@pytest.fixture(autouse=True)
def _clean(monkeypatch):
    monkeypatch.delenv("MABA_BACKEND", raising=False)
    D.clear_fallback_warnings()
    yield
    D.clear_fallback_warnings()


@pytest.mark.parametrize("env,exp", [("hip", "hip"), ("triton", "hip"), ("cuda", "hip"), ("gpu", "hip"),
                                     ("cpu", "cpu"), ("openmp", "cpu"), ("reference", "reference"),
                                     ("pytorch", "reference"), ("ref", "reference"), ("xla", "xla"),
                                     ("tpu", "xla"), ("AUTO", "cpu")])
def test_env_override(monkeypatch, env, exp):
    monkeypatch.setenv("MABA_BACKEND", env)
    assert D.get_backend(torch.device("cpu")) == exp


def test_rocm_is_not_a_backend_name(monkeypatch):
    """The reference rejects unknown names (tests/test_dispatcher_fallbacks.py:212-249)."""
    monkeypatch.setenv("MABA_BACKEND", "rocm")
    with pytest.raises(ValueError, match="Unsupported MABA_BACKEND 'rocm'"):
        D.get_backend(torch.device("cpu"))


def test_auto_routing():
    assert D.get_backend(torch.device("cpu")) == "cpu"
    assert D.get_backend("cpu") == "cpu"
    assert D.get_backend(torch.device("meta")) == "reference"
    cuda = D.get_backend(torch.device("cuda", 0))
    assert cuda == ("hip" if torch.version.hip else "reference")


def test_backend_cache_keyed_by_env(monkeypatch):
    assert D.get_backend("cpu") == "cpu"
    monkeypatch.setenv("MABA_BACKEND", "reference")
    assert D.get_backend("cpu") == "reference"


def test_register_kernel_creates_backend_and_op():
    @D.register_kernel("unit_test_backend", "unit_test_op")
    def fn(**kw):
        return 42
    try:
        assert D.get_kernel("unit_test_backend", "unit_test_op") is fn
        assert D.get_kernel("unit_test_backend", "missing") is None
    finally:
        D._KERNEL_REGISTRY.pop("unit_test_backend")


def test_hip_backend_registers_every_op():
    for op in ("dgda_prefill", "dgda_step", "compute_centroids", "index_topk", "stream_superposition",
               "index_topk_decode", "hca_pool", "maba_sa_decode", "dgda_prologue",
               "maba_sa_prefill"):
        assert D.get_kernel("hip", op) is not None, op


def _swap(op, fn):
    old = D._KERNEL_REGISTRY["cpu"].get(op)
    D._KERNEL_REGISTRY["cpu"][op] = fn
    return old


def test_fallback_warns_once_and_runs_reference(monkeypatch):
    monkeypatch.setenv("MABA_STRICT_BACKEND", "0")

    def boom(**kw):
        raise ValueError("boom")
    old = _swap("compute_centroids", boom)
    try:
        k = torch.randn(2, 100, 8)
        with warnings.catch_warnings(record=True) as rec:
            warnings.simplefilter("always")
            c1 = D.dispatch_compute_centroids(k, block_size=64)
            c2 = D.dispatch_compute_centroids(k, block_size=64)
        msgs = [str(w.message) for w in rec if issubclass(w.category, RuntimeWarning)]
        assert len(msgs) == 1
        for part in ("compute_centroids", "'cpu'", "ValueError: boom", "Falling back to reference"):
            assert part in msgs[0]
        ref = C.ref_compute_centroids(k, block_size=64)
        assert torch.equal(c1, ref) and torch.equal(c2, ref)
    finally:
        _swap("compute_centroids", old)


def test_strict_mode_raises(monkeypatch):
    monkeypatch.setenv("MABA_STRICT_BACKEND", "1")

    def boom(**kw):
        raise RuntimeError("kernel failed")
    old = _swap("stream_superposition", boom)
    try:
        x = torch.randn(1, 2, 4, 8)
        with pytest.raises(RuntimeError, match="Falling back to reference"):
            D.dispatch_stream_superposition(x, x, x, gate_logits=torch.randn(1, 4, 3))
    finally:
        _swap("stream_superposition", old)


def test_missing_hip_library_is_never_papered_over(monkeypatch):
    monkeypatch.setenv("MABA_STRICT_BACKEND", "0")

    def missing(**kw):
        raise HipLibraryMissing("libmaba_hip.so not built")
    old = _swap("hca_pool", missing)
    try:
        with pytest.raises(HipLibraryMissing):
            D.dispatch_hca_pool(torch.randn(1, 128, 8), pool=64)
    finally:
        _swap("hca_pool", old)


def test_dgda_dtype_contract():
    B, H, L, d = 1, 2, 5, 4
    q = torch.randn(B, H, L, d, dtype=torch.bfloat16)
    g = torch.rand(B, H, L, d)
    with pytest.raises(TypeError, match="dtypes must match"):
        D.dispatch_dgda_prefill(q, q, q, alpha=g, b=g, w=g)
    with pytest.raises(ValueError, match="alpha or log_alpha"):
        D.dispatch_dgda_prefill(q, q, q, b=q, w=q)
    with pytest.raises(TypeError, match="Unsupported dtype"):
        D.dispatch_dgda_prefill(q.int(), q.int(), q.int(), alpha=g, b=g, w=g)


def test_dispatch_matches_reference_on_cpu():
    torch.manual_seed(0)
    B, H, L, d = 1, 2, 40, 8
    q = torch.nn.functional.normalize(torch.randn(B, H, L, d), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, H, L, d), dim=-1)
    v = torch.randn(B, H, L, d)
    la = -torch.nn.functional.softplus(torch.randn(B, H, L, d) + 2)
    beta = torch.sigmoid(torch.randn(B, H, L, d))
    # the cpu backend's chunked form with the reference's adaptive inversion (series, then the
    # exact solve where the residual exceeds the tolerance) against the token loop
    o, S = D.dispatch_dgda_prefill(q, k, v, b=beta, w=beta, log_alpha=la, chunk_size=16,
                                   inversion_method="adaptive", adaptive_tol=1e-6)
    o2, S2 = C.ref_dgda_prefill(q, k, v, b=beta, w=beta, log_alpha=la)
    assert torch.allclose(o, o2, atol=1e-5) and torch.allclose(S, S2, atol=1e-5)


def test_hip_wrappers_refuse_cpu_tensors_and_autograd():
    from maba_sparse.kernels import hip_backend as hb
    x = torch.randn(1, 128, 64)
    with pytest.raises(RuntimeError, match="GPU tensors"):
        hb.hip_compute_centroids(x, block_size=64)
    xr = x.clone().requires_grad_(True)
    with pytest.raises(NotImplementedError):
        hb.hip_compute_centroids(xr, block_size=64)


def test_concurrent_dispatch_from_threads():
    """Callers may come from several Python threads (test_dispatcher_fallbacks.py:251-294)."""
    k = torch.randn(2, 256, 16)
    ref = C.ref_compute_centroids(k, block_size=64)
    errors = []

    def work():
        try:
            for _ in range(20):
                D.clear_dispatcher_cache()
                assert torch.equal(D.dispatch_compute_centroids(k, block_size=64), ref)
        except Exception as e:  # noqa: BLE001
            errors.append(e)
    ts = [threading.Thread(target=work) for _ in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors


def test_maba_sa_decode_reference_matches_explicit_streams():
    """The dispatcher's latent-space reference against a direct composition of
    per-stream softmax attention with the gate (float64)."""
    torch.manual_seed(1)
    B, H, dc, L = 2, 3, 16, 300
    c = torch.randn(B, L, dc, dtype=torch.float64)
    q_lat = torch.randn(B, H, dc, dtype=torch.float64)
    hca = D.dispatch_hca_pool(c, pool=64)
    idx = torch.stack([torch.randperm(5)[:3] for _ in range(B)]).view(B, 1, 3)
    gate = torch.randn(B, 3, dtype=torch.float64)
    z = D.dispatch_maba_sa_decode(q_lat, c, hca, idx, gate, L=L, scale=0.25)
    g = torch.softmax(gate, -1)
    for b in range(B):
        loc = list(range(4)) + list(range(L - 128, L))
        sp = [p for blk in idx[b, 0].tolist() for p in range(64 * blk, 64 * blk + 64) if p < L]
        for h in range(H):
            out = torch.zeros(dc, dtype=torch.float64)
            for s, rows in enumerate((c[b, loc], c[b, sp], hca[b])):
                p = torch.softmax(rows @ q_lat[b, h] * 0.25, 0)
                out += g[b, s] * (p @ rows)
            assert torch.allclose(z[b, h].double(), out, rtol=1e-5, atol=1e-5), (b, h)   # fp32 result


def test_maba_sa_prefill_reference_matches_oracle():
    """The dispatcher's torch prefill (the CPU path and the fallback) against the oracle's
    dense-mask restatement, with a past (Lq < Lkv), early rows, a shared index row and a
    repeated block."""
    import numpy as np
    from oracle import sparse_attn as osa
    g = torch.Generator().manual_seed(3)
    B, H, Lq, Lkv, dh, K = 2, 3, 90, 150, 8, 4
    q = torch.randn(B, H, Lq, dh, generator=g, dtype=torch.float64)
    k, v = (torch.randn(B, H, Lkv, dh, generator=g, dtype=torch.float64) for _ in range(2))
    kh, vh = (torch.randn(B, H, Lkv // 64, dh, generator=g, dtype=torch.float64) for _ in range(2))
    early = torch.randn(B, H, 3, dh, generator=g, dtype=torch.float64)     # pos 60..62 < 63
    gate = torch.randn(B, Lq, 3, generator=g, dtype=torch.float64)
    for idx in (torch.randint(0, 3, (B, Lq, K), generator=g), torch.tensor([[[0, 2, 2, 1]], [[1, 1, 0, 0]]])):
        got = D.dispatch_maba_sa_prefill(q, k, v, kh, vh, early, idx, gate, scale=0.3, window=40, n_sink=2)
        exp = osa.maba_sa_prefill_heads(q.numpy(), k.numpy(), v.numpy(), kh.numpy(), vh.numpy(), early.numpy(),
                                        idx.numpy(), gate.numpy(), window=40, n_sink=2, scale=0.3)
        assert np.allclose(got.numpy(), exp, rtol=1e-10, atol=1e-12)
