"""Kernels of the device-resident decode step, on the GPU.

- ``cache_append`` against ``oracle.indexer.decode_centroid_cache`` and
  ``oracle.sparse_attn.hca_means`` after every appended token, across block boundaries
  (centroids and means within half a bf16 ulp of the float64 values, plus fp32 slack;
  appended rows bit-exact).
- ``index_topk_decode_dev`` / ``maba_sa_decode_dev`` (length in device memory, buffers of
  fixed capacity) against the host-length entry points on the same rows: indices
  bit-exact, latent outputs within 1e-5, and the MABA-SA output within the north-star 2e-3
  of the float64 oracle.
- ``rmsnorm`` (with and without the gated residual) and ``swiglu`` against float64 torch
  on the same bf16 inputs: one bf16 rounding of the result (half an ulp plus fp32 slack).
- the DGDA step with a bf16 state (in place and out of place) and the single-token
  prologue (in-place history) against the float64 oracle.
"""
import math

import numpy as np
import pytest
import torch

from _helpers import assert_close, to_np
from oracle import dgda as odgda
from oracle import indexer as oidx
from oracle import sparse_attn as osa

pytestmark = pytest.mark.gpu


def _hb():
    from maba_sparse.kernels import hip_backend
    return hip_backend


def _ulp_close(got, exp, what):
    g = to_np(got)
    e = np.asarray(exp, np.float64)
    bound = (2.0 ** -8 + 1e-5) * np.abs(e) + 1e-6
    bad = np.abs(g - e) > bound
    assert not bad.any(), f"{what}: {bad.sum()} values beyond half a bf16 ulp (max err {np.abs(g - e).max():.3e})"


def test_cache_append_vs_oracle(dev):
    hb = _hb()
    g = torch.Generator().manual_seed(3)
    B, dc, di, Lmax, L0, steps = 3, 128, 64, 320, 100, 170       # crosses 128, 192, 256
    c_all = torch.randn(B, Lmax, dc, generator=g).bfloat16()
    k_all = torch.randn(B, Lmax, di, generator=g).bfloat16()
    c = torch.zeros(B, Lmax, dc, dtype=torch.bfloat16, device=dev)
    k = torch.zeros(B, Lmax, di, dtype=torch.bfloat16, device=dev)
    hca = torch.zeros(B, Lmax // 64, dc, dtype=torch.bfloat16, device=dev)
    cent = torch.zeros(B, (Lmax + 63) // 64, di, dtype=torch.bfloat16, device=dev)
    c[:, :L0] = c_all[:, :L0].to(dev)
    k[:, :L0] = k_all[:, :L0].to(dev)
    hca[:, : L0 // 64] = hb.hip_hca_pool(c[:, :L0], pool=64)
    cent[:, : L0 // 64] = hb.hip_compute_centroids(k[:, : (L0 // 64) * 64], block_size=64)
    pos = torch.tensor([L0], dtype=torch.long, device=dev)
    for t in range(L0, L0 + steps):
        hb.hip_cache_append(c_all[:, t].to(dev), k_all[:, t].to(dev), pos[0], c, k, hca, cent)
        pos += 1
        n = t + 1
        assert torch.equal(c[:, t].cpu(), c_all[:, t]) and torch.equal(k[:, t].cpu(), k_all[:, t])
        if n % 64 == 0 or n % 37 == 0 or t == L0 + steps - 1:
            _ulp_close(hca[:, : n // 64], osa.hca_means(to_np(c_all[:, :n]), n, 64), f"hca means at n={n}")
            _ulp_close(cent[:, : (n + 63) // 64], oidx.decode_centroid_cache(to_np(k_all[:, :n]), 64),
                       f"centroid cache at n={n}")
    assert int(pos) == L0 + steps


@pytest.mark.parametrize("L", [2048 + 5, 6400, 25000])
def test_index_topk_decode_dev_matches_host(dev, L):
    hb = _hb()
    g = torch.Generator().manual_seed(L)
    B, Hq, d, ncap = 4, 3, 64, 400
    cent = torch.randn(B, ncap, d, generator=g).bfloat16().to(dev)
    q = torch.randn(B, Hq, d, generator=g).bfloat16().to(dev)
    nb = (L + 63) // 64
    length = torch.tensor([L], dtype=torch.long, device=dev)
    got = hb.hip_index_topk_decode_dev(q, cent, length[0], 64, 0.1, 32)
    exp = hb.hip_index_topk_decode(q, cent[:, :nb], lambda_dist=0.1, top_k=32)
    assert torch.equal(got, exp)


@pytest.mark.parametrize("L,Hi", [(700, 1), (5000, 4), (19999, 1), (20000, 4)])
def test_maba_sa_decode_dev_matches_host(dev, L, Hi):
    hb = _hb()
    g = torch.Generator().manual_seed(L + Hi)
    B, H, dh, dc, Lcap, K = 2, 4, 64, 128, 20000, 16
    c = torch.randn(B, Lcap, dc, generator=g).bfloat16()
    Wk = torch.randn(H * dh, dc, generator=g) * 0.05
    Wv = torch.randn(H * dh, dc, generator=g) * 0.05
    q = torch.randn(B, H, dh, generator=g)
    nb = (L + 63) // 64
    idx = torch.stack([torch.stack([torch.randperm(nb, generator=g)[:K] for _ in range(Hi)]) for _ in range(B)])
    gate = torch.randn(B, 3, generator=g)
    cd = c.to(dev)
    hca = torch.zeros(B, Lcap // 64, dc, dtype=torch.bfloat16, device=dev)
    hca[:, : L // 64] = hb.hip_hca_pool(cd[:, :L], pool=64)
    q_lat = torch.einsum("bhd,hdc->bhc", q, Wk.view(H, dh, dc)).to(dev)
    length = torch.tensor([L], dtype=torch.long, device=dev)
    z_dev = hb.hip_maba_sa_decode_dev(q_lat, cd, hca, idx.to(dev), gate.to(dev), length[0], Lcap, 1 / math.sqrt(dh))
    z_host = hb.hip_maba_sa_decode(q_lat, cd, hca[:, : max(L // 64, 1)], idx.to(dev), gate.to(dev), L=L,
                                   scale=1 / math.sqrt(dh))
    assert_close(z_dev, to_np(z_host), 1e-5, 1e-6, "device-length decode vs host length")
    out = torch.einsum("bhc,hdc->bhd", z_dev.cpu(), Wv.view(H, dh, dc))
    exp = osa.maba_sa_decode(to_np(q), to_np(c[:, :L]), to_np(Wk), to_np(Wv), to_np(idx).astype(np.int64),
                             to_np(gate))
    assert_close(out, exp, 2e-3, 2e-3, "device-length decode vs oracle")


@pytest.mark.parametrize("rows,C,dtype", [((16, 1), 640, torch.bfloat16), ((3, 70), 640, torch.bfloat16),
                                          ((5, 1), 1248, torch.float32), ((2, 9), 96, torch.bfloat16)])
def test_rmsnorm_and_residual(dev, rows, C, dtype):
    hb = _hb()
    g = torch.Generator().manual_seed(C)
    x = torch.randn(*rows, C, generator=g).to(dtype)
    mo = torch.randn(*rows, C, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(C, generator=g)).to(dtype)
    gate = torch.sigmoid(torch.randn(C, generator=g)).to(dtype)
    eps = 1e-6
    h = hb.hip_rmsnorm(x.to(dev), w.to(dev), eps)
    xd = x.double()
    ref = xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + eps) * w.double()
    _ulp_close(h, ref.numpy(), "rmsnorm") if dtype == torch.bfloat16 else assert_close(h, ref.numpy(), 1e-5, 1e-6, "rmsnorm")
    xo = torch.empty_like(x, device=dev)
    h2 = hb.hip_rmsnorm(x.to(dev), w.to(dev), eps, mo=mo.to(dev), gate=gate.to(dev), x_out=xo)
    xr = (x.double() + gate.double() * mo.double())
    if dtype == torch.bfloat16:
        _ulp_close(xo, xr.numpy(), "gated residual")
    xs = xo.cpu().double()                                   # the norm reads the stored residual
    ref2 = xs / torch.sqrt((xs * xs).mean(-1, keepdim=True) + eps) * w.double()
    _ulp_close(h2, ref2.numpy(), "rmsnorm of the residual") if dtype == torch.bfloat16 else \
        assert_close(h2, ref2.numpy(), 1e-5, 1e-6, "rmsnorm of the residual")
    # the residual without x_out is normalised unrounded; gate and weight of the other dtype
    other = torch.float32 if dtype == torch.bfloat16 else torch.bfloat16
    w3, g3 = w.to(other), gate.to(other)
    h3 = hb.hip_rmsnorm(x.to(dev), w3.to(dev), eps, mo=mo.to(dev), gate=g3.to(dev))
    xr3 = x.double() + g3.double() * mo.double()
    ref3 = xr3 / torch.sqrt((xr3 * xr3).mean(-1, keepdim=True) + eps) * w3.double()
    _ulp_close(h3, ref3.numpy(), "rmsnorm of the unstored residual") if dtype == torch.bfloat16 else \
        assert_close(h3, ref3.numpy(), 1e-5, 1e-6, "rmsnorm of the unstored residual")
    xo4 = x.clone().to(dev)                                  # x_out aliasing x, mixed dtypes
    h4 = hb.hip_rmsnorm(xo4, w3.to(dev), eps, mo=mo.to(dev), gate=g3.to(dev), x_out=xo4)
    xs4 = xo4.cpu().double()
    if dtype == torch.bfloat16:
        _ulp_close(xo4, xr3.numpy(), "gated residual in place")
    ref4 = xs4 / torch.sqrt((xs4 * xs4).mean(-1, keepdim=True) + eps) * w3.double()
    _ulp_close(h4, ref4.numpy(), "rmsnorm in place") if dtype == torch.bfloat16 else \
        assert_close(h4, ref4.numpy(), 1e-5, 1e-6, "rmsnorm in place")


@pytest.mark.parametrize("shape,dtype", [((16, 1, 2496), torch.bfloat16), ((3, 50, 96), torch.float32)])
def test_swiglu(dev, shape, dtype):
    hb = _hb()
    gu = torch.randn(*shape, generator=torch.Generator().manual_seed(shape[-1])).to(dtype)
    out = hb.hip_swiglu(gu.to(dev))
    I = shape[-1] // 2
    gd, ud = gu[..., :I].double(), gu[..., I:].double()
    ref = gd / (1 + torch.exp(-gd)) * ud
    if dtype == torch.bfloat16:
        _ulp_close(out, ref.numpy(), "swiglu")
    else:
        assert_close(out, ref.numpy(), 1e-5, 1e-6, "swiglu")


def test_swiglu_row_kernel_matches_generic(dev):
    """bf16 rows of 16-byte aligned width take the one-wave-per-row kernel; the same rows at
    a 4-byte offset (not 16-byte aligned) take the element-pair kernel: equal bits."""
    hb = _hb()
    shape = (3, 333, 2 * 1248)
    gu = torch.randn(*shape, generator=torch.Generator().manual_seed(9)).bfloat16().to(dev)
    out = hb.hip_swiglu(gu)
    buf = torch.empty(gu.numel() + 8, dtype=torch.bfloat16, device=dev)
    shifted = buf[2: 2 + gu.numel()].view(shape)
    shifted.copy_(gu)
    assert shifted.data_ptr() % 16 != 0
    assert torch.equal(hb.hip_swiglu(shifted), out)
    I = shape[-1] // 2
    gd, ud = gu[..., :I].double().cpu(), gu[..., I:].double().cpu()
    _ulp_close(out, (gd / (1 + torch.exp(-gd)) * ud).numpy(), "swiglu rows")


@pytest.mark.parametrize("inplace", [False, True])
def test_dgda_step_bf16_state(dev, inplace):
    hb = _hb()
    g = torch.Generator().manual_seed(7)
    B, H, d = 16, 10, 64
    q = torch.nn.functional.normalize(torch.randn(B, H, d, generator=g), dim=-1).bfloat16()
    k = torch.nn.functional.normalize(torch.randn(B, H, d, generator=g), dim=-1).bfloat16()
    v = torch.randn(B, H, d, generator=g).bfloat16()
    la = -torch.nn.functional.softplus(torch.randn(B, H, d, generator=g))
    b = torch.sigmoid(torch.randn(B, H, d, generator=g))
    w = torch.sigmoid(torch.randn(B, H, d, generator=g))
    S = (torch.randn(B, H, d, d, generator=g) * 0.3).bfloat16()
    Sd = S.to(dev)
    kw = dict(new_state=Sd) if inplace else {}
    o, Sn = hb.hip_dgda_step(q.to(dev), k.to(dev), v.to(dev), log_alpha=la.to(dev), b=b.to(dev), w=w.to(dev),
                             state=Sd, allow_mixed_dtypes=True, out_dtype=torch.float32, **kw)
    if inplace:
        assert Sn.data_ptr() == Sd.data_ptr()
    eo, eS = odgda.dgda_step(to_np(q), to_np(k), to_np(v), alpha=np.exp(to_np(la)), b=to_np(b), w=to_np(w),
                             state=to_np(S))
    assert Sn.dtype == torch.bfloat16
    assert_close(o, eo, 1e-4, 1e-4, "step output (fp32 from the bf16 state)")
    _ulp_close(Sn, eS, "bf16 state")


@pytest.mark.parametrize("hist_dtype", [torch.float32, torch.bfloat16])
def test_prologue_single_token_in_place(dev, hist_dtype):
    hb = _hb()
    g = torch.Generator().manual_seed(11)
    B, H = 16, 10
    C = 64 * H
    xs = [torch.randn(B, 1, C, generator=g).bfloat16() for _ in range(6)]
    cw = [(torch.randn(C, 1, 4, generator=g) * 0.5).bfloat16() for _ in range(3)]
    hist = [torch.randn(B, C, 3, generator=g).to(hist_dtype) for _ in range(3)]
    hd = [h.to(dev) for h in hist]
    outs = hb.hip_dgda_prologue([x.to(dev) for x in xs], [w.to(dev) for w in cw], history=hd, n_heads=H,
                                eps=1e-6, gate_dtype=torch.float32, with_alpha=False, out_history=hd)
    q, k, v, la, _, b, w, nh = outs
    assert all(a.data_ptr() == c.data_ptr() for a, c in zip(nh, hd))
    eq, ek, ev, ela, _, eb, ew, enh = odgda.layer_prologue(*[to_np(x) for x in xs], *[to_np(c)[:, 0, :] for c in cw],
                                                           hist=[to_np(h) for h in hist], n_heads=H, eps=1e-6)
    for name, got, e in (("q", q, eq), ("k", k, ek), ("v", v, ev)):
        _ulp_close(got, e, f"single-token prologue {name}")
    assert_close(la, ela, 1e-5, 1e-6, "log_alpha")
    assert_close(b, eb, 1e-5, 1e-6, "erase gate")
    assert_close(w, ew, 1e-5, 1e-6, "write gate")
    for s in range(3):
        assert_close(nh[s], enh[s], 0, 0, f"new history {s}")


def test_maba_sa_device_decode_vs_oracle(dev):
    """A bf16 MABA-SA layer at the 101M widths: prefill 2,100 tokens, then 70 decode tokens on
    the device path (DeviceCache appends, device-length indexer and decode), crossing the
    block boundaries at 2,112 and 2,176.  At several steps the output is checked against the
    float64 oracle on the device cache's rows with oracle-computed means (2e-3), and the
    indexer's picks against oracle scores of the centroids the cache holds."""
    from maba_sparse.layers import MabaSparseAttention
    from maba_sparse.layers.sparse_attention import DeviceCache
    torch.manual_seed(5)
    B, L0, steps = 4, 2100, 70
    layer = MabaSparseAttention(dim=640, n_heads=10, d_head=64, d_c=128, d_idx=64, top_k=32,
                                dist_lambda=0.1).eval()
    with torch.no_grad():
        for p in layer.parameters():
            p.normal_(0.0, 0.05) if p.dim() > 1 else None
    layer = layer.to(dev, torch.bfloat16)
    g = torch.Generator().manual_seed(6)
    xs = torch.randn(B, L0 + steps, 640, generator=g).bfloat16().to(dev)
    with torch.no_grad():
        _, c_full = layer(xs[:, :L0])
        cache = DeviceCache(c_full, layer.indexer._cached_k_idx, L0 + steps)
        counters = torch.tensor([L0, L0 + 1], dtype=torch.long, device=dev)
        for t in range(L0, L0 + steps):
            x = xs[:, t:t + 1]
            out, idx, z = layer.decode_step_device(x, cache, counters, return_parts=True)
            counters += 1
            L = t + 1
            if t - L0 in (0, 11, 12, 13, 45, 69):
                q, _, qi, _, gl = layer._token_projections(x)
                nb = (L + 63) // 64
                ref_sc = oidx.decode_scores(to_np(qi), oidx.decode_centroid_cache(to_np(cache.keys[:, :L]), 64), 0.1)
                from _helpers import topk_is_valid
                topk_is_valid(idx.cpu().numpy(), ref_sc, 2e-2)          # centroids are bf16-rounded
                assert idx.shape == (B, 1, 32) and int(idx.max()) < nb
                got = torch.einsum("bhc,hdc->bhd", z.cpu(), layer.v_up_proj.weight.float().cpu().view(10, 64, 128))
                exp = osa.maba_sa_decode(to_np(q.view(B, 10, 64)), to_np(cache.c[:, :L]),
                                         to_np(layer.k_up_proj.weight), to_np(layer.v_up_proj.weight),
                                         to_np(idx).astype(np.int64), to_np(gl.view(-1, 3)), L=L)
                assert_close(got, exp, 2e-3, 2e-3, f"device decode at L={L}")


def test_cache_append_heads_and_value_up(dev):
    """The serving step's fused extras: ``cache_append_heads`` appends like ``cache_append``
    (bit-exact caches) and forms ``q_lat = W_k,h^T q_h`` (float64 reference, fp32 slack) and
    ``bf16(gate + bias)`` (exact); ``maba_sa_decode_dev_heads`` returns the same ``z`` as
    ``maba_sa_decode_dev`` (bit-exact: same kernels) and ``W_v,h z_h`` rounded to bf16 within
    half an ulp of the float64 product of that ``z``."""
    hb = _hb()
    g = torch.Generator().manual_seed(11)
    B, L0, cap, H, dh, dc, di = 3, 700, 800, 10, 64, 128, 64
    bf = torch.bfloat16
    c_all = torch.randn(B, L0 + 1, dc, generator=g).to(bf)
    k_all = torch.randn(B, L0 + 1, di, generator=g).to(bf)

    def caches():
        c = torch.zeros(B, cap, dc, dtype=bf, device=dev)
        k = torch.zeros(B, cap, di, dtype=bf, device=dev)
        c[:, :L0] = c_all[:, :L0].to(dev)
        k[:, :L0] = k_all[:, :L0].to(dev)
        hca = torch.zeros(B, cap // 64, dc, dtype=bf, device=dev)
        hca[:, : L0 // 64] = hb.hip_hca_pool(c[:, : (L0 // 64) * 64])
        cent = torch.zeros(B, (cap + 63) // 64, di, dtype=bf, device=dev)
        cent[:, : (L0 + 63) // 64] = hb.hip_compute_centroids(k[:, :L0])
        return c, k, hca, cent

    qh = torch.randn(B, 1, H * dh, generator=g).to(bf).to(dev)
    wk = (0.05 * torch.randn(H * dh, dc, generator=g)).to(bf).to(dev)
    wv = (0.05 * torch.randn(H * dh, dc, generator=g)).to(bf).to(dev)
    gin = torch.randn(B, 1, 3, generator=g).to(bf).to(dev)
    gbias = torch.randn(3, generator=g).to(bf).to(dev)
    pos = torch.tensor([L0, L0 + 1], dtype=torch.long, device=dev)
    c1, k1, hca1, cent1 = caches()
    c2, k2, hca2, cent2 = caches()
    cn, kn = c_all[:, L0].to(dev), k_all[:, L0].to(dev)
    hb.hip_cache_append(cn, kn, pos[0], c1, k1, hca1, cent1)
    q_lat = torch.empty(B, H, dc, dtype=torch.float32, device=dev)
    gate = torch.empty(B, 3, dtype=bf, device=dev)
    hb.hip_cache_append_heads(cn, kn, pos[0], c2, k2, hca2, cent2, qh[:, 0], wk, gin[:, 0], gbias, q_lat, gate)
    for x, y, what in ((c1, c2, "latent rows"), (k1, k2, "keys"), (hca1, hca2, "means"), (cent1, cent2, "centroids")):
        assert torch.equal(x, y), what
    q64 = qh[:, 0].double().cpu().view(B, H, dh)
    exp = torch.einsum("bhd,hdc->bhc", q64, wk.double().cpu().view(H, dh, dc))
    scale = torch.einsum("bhd,hdc->bhc", q64.abs(), wk.double().cpu().abs().view(H, dh, dc))
    assert ((q_lat.double().cpu() - exp).abs() <= 1e-6 * scale + 1e-9).all(), "absorbed query"
    assert torch.equal(gate.cpu(), (gin[:, 0] + gbias).cpu()), "gate logits + bias"

    idx = torch.randint(0, (L0 + 1) // 64, (B, 1, 32), generator=g).to(dev)
    z1 = hb.hip_maba_sa_decode_dev(q_lat, c2, hca2, idx, gate, pos[1], cap, 1 / math.sqrt(dh))
    o = torch.empty(B, H * dh, dtype=bf, device=dev)
    z2 = hb.hip_maba_sa_decode_dev_heads(q_lat, c2, hca2, idx, gate, pos[1], cap, 1 / math.sqrt(dh), wv, o)
    assert torch.equal(z1, z2), "z"
    o_exp = torch.einsum("bhc,hdc->bhd", z2.double().cpu(), wv.double().cpu().view(H, dh, dc)).reshape(B, H * dh)
    _ulp_close(o, o_exp, "value up-projection")


def test_serving_layer_step_fused_heads_matches_unfused(dev, monkeypatch):
    """``decode_step_device`` with the fused extras against the same step with the separate
    torch launches (absorbed query, gate bias, value up-projection): identical selections, ``z``
    within 1e-4 (the absorbed query's fp32 sums run in another order, and the softmax carries
    that through) and the layer outputs within two bf16 ulps of the output scale."""
    from maba_sparse.layers import MabaSparseAttention
    from maba_sparse.layers.sparse_attention import DeviceCache
    torch.manual_seed(7)
    B, L0, steps = 4, 2100, 8   # the device-length indexer needs at least top_k blocks
    layer = MabaSparseAttention(dim=640, n_heads=10, d_head=64, d_c=128, d_idx=64, top_k=32,
                                dist_lambda=0.1).eval()
    with torch.no_grad():
        for p in layer.parameters():
            p.normal_(0.0, 0.05) if p.dim() > 1 else p.normal_(0.0, 0.5)
    layer = layer.to(dev, torch.bfloat16)
    assert layer._heads_fusable()
    g = torch.Generator().manual_seed(8)
    xs = torch.randn(B, L0 + steps, 640, generator=g).bfloat16().to(dev)
    with torch.no_grad():
        _, c_full = layer(xs[:, :L0])
        keys = layer.indexer._cached_k_idx
        ca = DeviceCache(c_full, keys, L0 + steps)
        cb = DeviceCache(c_full, keys, L0 + steps)
        cnt_a = torch.tensor([L0, L0 + 1], dtype=torch.long, device=dev)
        cnt_b = cnt_a.clone()
        for t in range(L0, L0 + steps):
            x = xs[:, t:t + 1]
            oa, ia, za = layer.decode_step_device(x, ca, cnt_a, return_parts=True)
            with monkeypatch.context() as m:
                m.setattr(type(layer), "_heads_fusable", lambda self: False)
                ob, ib, zb = layer.decode_step_device(x, cb, cnt_b, return_parts=True)
            cnt_a += 1
            cnt_b += 1
            assert torch.equal(ia, ib), f"selections at {t}"
            assert_close(za, to_np(zb), 1e-4, 1e-5, f"z at {t}")   # q_lat summed in another order
            sc = ob.float().abs().max().item()
            assert (oa.float() - ob.float()).abs().max().item() <= 2 * 2.0 ** -8 * sc, f"output at {t}"


def _dl_case(M, K, N, mode, seed):
    """Inputs of one decode_linear case and the float64 product of its bf16 operand A."""
    g = torch.Generator().manual_seed(seed)
    bf = torch.bfloat16
    a = torch.randn(M, 1, 2 * K if mode == "swiglu" else K, generator=g).to(bf)
    w = (torch.randn(N, K, generator=g) / math.sqrt(K)).to(bf)
    mo = torch.randn(M, 1, K, generator=g).to(bf)
    gate = torch.sigmoid(torch.randn(K, generator=g)).to(bf)
    nw = (1 + 0.1 * torch.randn(K, generator=g)).to(bf)
    return a, w, mo, gate, nw


def _dl_ref(A, w):
    """A [M, K] (float64 values of the bf16 operand) times w^T, and the absolute-sum scale."""
    wd = w.double()
    return A @ wd.T, A.abs() @ wd.abs().T


def _bf16(x):
    return x.to(torch.bfloat16).double()


@pytest.mark.parametrize("M,K,N,mode", [
    (16, 640, 640, "plain"), (3, 128, 200, "plain"), (20, 1248, 48, "plain"), (16, 640, 3840, "norm"),
    (16, 640, 2496, "normres"), (5, 96, 40, "normres"), (16, 1024, 32, "normres"), (4, 2048, 48, "norm"),
    (16, 1248, 640, "swiglu"), (7, 2048, 64, "swiglu"), (3, 4096, 32, "plain")])
def test_decode_linear_modes(dev, M, K, N, mode):
    """y = A W^T with A's input stage in the same launch, against float64 on the same bf16
    operand: the output is one bf16 rounding (half an ulp) of the product; an element of A
    that the kernel (fp32, then bf16) and float64 round to neighbouring bf16 values moves y
    by at most an ulp of that one term, inside 1e-3 of the absolute-sum scale.  y and x_out
    are views into larger buffers whose other elements must stay untouched."""
    hb = _hb()
    a, w, mo, gate, nw = _dl_case(M, K, N, mode, seed=K + N + M)
    ybuf = torch.full((M + 2, 1, N + 16), 7.0, dtype=torch.bfloat16, device=dev)
    y = ybuf[:M, :, :N]
    xbuf = torch.full((M + 1, 1, K), 7.0, dtype=torch.bfloat16, device=dev)
    kw = {}
    if mode == "norm":
        kw = dict(norm_w=nw.to(dev))
    elif mode == "normres":
        kw = dict(norm_w=nw.to(dev), mo=mo.to(dev), gate=gate.to(dev), x_out=xbuf[:M])
    hb.hip_decode_linear(a.to(dev), w.to(dev), eps=1e-6, swiglu=mode == "swiglu", out=y, **kw)
    torch.cuda.synchronize()
    ad = a[:, 0].double()
    if mode == "plain":
        A, slack = ad, 1e-5
    elif mode == "swiglu":
        gg, uu = ad[:, :K], ad[:, K:]
        A, slack = _bf16(gg * torch.sigmoid(gg) * uu), 1e-3
    else:
        x = ad
        if mode == "normres":
            xr = ad + gate.double() * mo[:, 0].double()
            xo = xbuf[:M, 0].cpu().double()
            _ulp_close(xo, xr.numpy(), "decode_linear x_out")
            assert torch.all(xbuf[M:].cpu() == 7.0), "x_out written past its rows"
            x = xo
        A, slack = _bf16(x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6) * nw.double()), 1e-3
    ref, scale = _dl_ref(A, w)
    got = y[:, 0].cpu().double()
    bad = (got - ref).abs() > 2.0 ** -8 * ref.abs() + slack * scale + 1e-6
    assert not bad.any(), f"{mode}: {int(bad.sum())} of {bad.numel()} beyond bound (max err {(got - ref).abs().max():.3e})"
    rest = ybuf.cpu().clone()
    rest[:M, :, :N] = 7.0
    assert torch.all(rest == 7.0), "y written outside its view"


def test_decode_linear_rejects(dev):
    hb = _hb()
    bf = torch.bfloat16
    a = torch.randn(4, 1, 640, device=dev).to(bf)
    w = torch.randn(64, 640, device=dev).to(bf)
    nw = torch.ones(640, device=dev, dtype=bf)
    with pytest.raises(Exception, match="multiple of 32"):
        hb.hip_decode_linear(a[..., :600], w[:, :600].contiguous())
    with pytest.raises(Exception, match="2048 with a norm"):
        hb.hip_decode_linear(torch.randn(4, 2080, device=dev).to(bf), torch.randn(8, 2080, device=dev).to(bf),
                             norm_w=torch.ones(2080, device=dev, dtype=bf))
    with pytest.raises(Exception, match="may not overlap"):
        hb.hip_decode_linear(a, w, norm_w=nw, mo=a.clone(), gate=nw, x_out=a)
    with pytest.raises(Exception, match="16-byte aligned"):
        buf = torch.randn(4, 648, device=dev).to(bf)
        hb.hip_decode_linear(buf[:, 1:641], w)
    # the output may not overlap the residual input or the residual written in the same launch
    mo, xo = a.clone(), torch.empty_like(a)
    with pytest.raises(Exception, match="y may not overlap mo or x_out"):
        hb.hip_decode_linear(a, w, norm_w=nw, mo=mo, gate=nw, x_out=xo, out=mo[..., :64])
    with pytest.raises(Exception, match="y may not overlap mo or x_out"):
        hb.hip_decode_linear(a, w, norm_w=nw, mo=mo, gate=nw, x_out=xo, out=xo[..., 64:128])


def test_rmsnorm_and_cache_append_reject_empty_axes(dev):
    """An empty channel axis for the norm, and an absorbed-query buffer with no heads for the
    fused append, are argument errors raised before anything launches."""
    hb = _hb()
    bf = torch.bfloat16
    with pytest.raises(ValueError, match="at least 2 channels"):
        hb.hip_rmsnorm(torch.empty(3, 0, device=dev, dtype=bf), torch.empty(0, device=dev, dtype=bf), 1e-6)
    B, cap, dc, di = 2, 128, 128, 64
    z = lambda *s: torch.zeros(*s, device=dev, dtype=bf)  # noqa: E731
    pos = torch.tensor([5, 6], dtype=torch.long, device=dev)
    with pytest.raises(ValueError, match="q_lat"):
        hb.hip_cache_append_heads(z(B, dc), z(B, di), pos[0], z(B, cap, dc), z(B, cap, di), z(B, cap // 64, dc),
                                  z(B, cap // 64, di), z(B, 640), z(640, dc), z(B, 3), z(3),
                                  torch.empty(B, 0, dc, device=dev), z(B, 3))


def test_decode_linear_gather(dev):
    """Table rows picked by int64 ids (the embedding lookup before its projection), ids
    outside the table clamped into it: equal to the plain decode linear on the gathered rows."""
    hb = _hb()
    g = torch.Generator().manual_seed(11)
    table = torch.randn(1000, 128, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(640, 128, generator=g) / 12).to(torch.bfloat16).to(dev)
    ids = torch.tensor([[5], [999], [0], [17], [5]], dtype=torch.long, device=dev)
    got = hb.hip_decode_linear(table, w, rows=ids)
    assert got.shape == (5, 1, 640)
    exp = hb.hip_decode_linear(table[ids[:, 0]].unsqueeze(1).contiguous(), w)
    assert torch.equal(got, exp)
    far = hb.hip_decode_linear(table, w, rows=torch.tensor([-3, 5000], dtype=torch.long, device=dev))
    assert torch.equal(far, hb.hip_decode_linear(table[[0, 999]].contiguous(), w))


@pytest.mark.parametrize("M,V,dtype", [(16, 32768, torch.bfloat16), (3, 1000, torch.float32), (2, 40000, torch.bfloat16)])
def test_argmax_rows(dev, M, V, dtype):
    """torch.argmax's pick, including ties (first index), -0 against +0, and NaN."""
    hb = _hb()
    g = torch.Generator().manual_seed(V)
    x = torch.randn(M, 1, V, generator=g).to(dtype)
    x[0, 0, [7, V - 3]] = 50.0                                    # a tie: the first wins
    if M > 1:
        x[1, 0, :] = -1.0
        x[1, 0, [V // 2, 3]] = torch.tensor([0.0, -0.0], dtype=dtype)   # -0 and +0 equal
    if M > 2:
        x[2, 0, [V - 1, 9]] = float("nan")                       # NaN is the maximum
    xd = x.to(dev)
    got = hb.hip_argmax_rows(xd)
    assert torch.equal(got.cpu(), xd.argmax(dim=-1).cpu())
    assert int(got[0, 0]) == 7
