"""The no-allocation MABA-SA decode entry point (``maba_hip_maba_sa_decode_static``) against
the workspace entry point (``maba_hip_maba_sa_decode``), both through the C ABI: two calls
in a row, the second smaller, each bit-identical to the workspace entry point's result
(same kernels and geometry) and within the north-star 2e-3 of the float64 oracle; a call
whose partials exceed the static scratch is refused before anything launches."""
import ctypes
import math

import numpy as np
import pytest
import torch

from _helpers import assert_close, to_np
from oracle import sparse_attn as osa

pytestmark = pytest.mark.gpu


def _case(dev, B, H, L, K, Hi, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    dh, dc = 64, 128
    c = torch.randn(B, L, dc, generator=g).to(dtype)
    Wk = torch.randn(H * dh, dc, generator=g) * 0.05
    Wv = torch.randn(H * dh, dc, generator=g) * 0.05
    q = torch.randn(B, H, dh, generator=g)
    nb = (L + 63) // 64
    idx = torch.stack([torch.stack([torch.randperm(nb, generator=g)[:min(K, nb)] for _ in range(Hi)])
                       for _ in range(B)])
    gate = torch.randn(B, 3, generator=g)
    q_lat = torch.einsum("bhd,hdc->bhc", q, Wk.view(H, dh, dc))
    return dict(c=c.to(dev), Wk=Wk, Wv=Wv, q=q, idx=idx.to(dev), gate=gate.to(dev), q_lat=q_lat.to(dev), L=L, H=H,
                dh=dh, dc=dc)


def _call(lib, N, cs, static):
    from maba_sparse.kernels import hip_backend as hb
    dev = cs["c"].device
    hca = hb.hip_hca_pool(cs["c"], pool=64)
    B, H, dc = cs["q_lat"].shape
    out = torch.full((B, H, dc), float("nan"), device=dev)
    args = [N.desc(cs["q_lat"]), N.desc(cs["c"]), N.desc(hca), N.desc(cs["idx"]), N.desc(cs["gate"]), int(cs["L"]),
            1.0 / math.sqrt(cs["dh"]), 128, 4, 64, 64, N.desc(out)]
    if static:
        rc = lib.maba_hip_maba_sa_decode_static(*args, N.stream_ptr(dev))
    else:
        K = cs["idx"].shape[-1]
        nbytes = lib.maba_hip_maba_sa_decode_workspace_size(B, H, dc, int(cs["L"]), K, 128, 4, 64)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        rc = lib.maba_hip_maba_sa_decode(*args, ws.data_ptr(), ws.numel(), N.stream_ptr(dev))
    N.check(rc, "maba_sa_decode_static" if static else "maba_sa_decode")
    torch.cuda.synchronize()
    return out, hca


def test_static_scratch_matches_workspace_entry(dev):
    from maba_sparse import _native as N
    lib = N.load()
    for B, H, L, K, Hi, seed in ((8, 10, 200_000, 32, 10, 1), (2, 4, 3000, 16, 1, 2)):   # second call smaller
        print(f"\nstatic decode B={B} H={H} L={L} K={K} Hi={Hi}", flush=True)
        cs = _case(dev, B, H, L, K, Hi, seed)
        z_static, hca = _call(lib, N, cs, static=True)
        z_ws, _ = _call(lib, N, cs, static=False)
        assert torch.equal(z_static, z_ws)
        out = torch.einsum("bhc,hdc->bhd", z_static.cpu(), cs["Wv"].view(H, cs["dh"], cs["dc"]))
        exp = osa.maba_sa_decode(to_np(cs["q"]), to_np(cs["c"]), to_np(cs["Wk"]), to_np(cs["Wv"]),
                                 to_np(cs["idx"]).astype(np.int64), to_np(cs["gate"]), means=to_np(hca))
        assert_close(out, exp, 2e-3, 2e-3, "static decode vs oracle")


def test_static_scratch_refuses_oversize(dev):
    """The per-tile path of an fp32 cache at B=4, H=16, L=200,000 needs about 19 MB of partials."""
    from maba_sparse import _native as N
    lib = N.load()
    cs = _case(dev, 4, 16, 200_000, 32, 16, 3, dtype=torch.float32)
    with pytest.raises(RuntimeError, match="static scratch"):
        _call(lib, N, cs, static=True)
