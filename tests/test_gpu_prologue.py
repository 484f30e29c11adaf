"""The DGDA layer prologue kernel (conv + SiLU with carried history, gates, key norm)
against the float64 oracle (``oracle.dgda.layer_prologue``) on seeded inputs.

Tolerances: fp32 outputs rtol 1e-5 / atol 1e-6 (fp32 arithmetic against float64);
bf16 outputs rtol 5e-3 / atol 1e-6 (one rounding to bf16: at most half an ulp, 2^-8
relative, on top of the fp32 error).  New histories are copies of inputs: exact.
"""
import numpy as np
import pytest
import torch

from _helpers import assert_close, to_np
from oracle import dgda as od

pytestmark = pytest.mark.gpu


def _hip():
    from maba_sparse.kernels import hip_backend
    return hip_backend


@pytest.mark.parametrize("B,L,H,dtype,with_hist,gdt", [
    (2, 1, 10, torch.float32, True, torch.float32),      # one decode token: all taps from the history
    (2, 2, 2, torch.float32, True, torch.float32),       # L < 3: the new history keeps the old one's tail
    (3, 37, 10, torch.float32, False, torch.float32),    # ragged last run of 16 tokens, zero history
    (2, 1000, 10, torch.bfloat16, True, torch.float32),  # the layer's bf16 path: fp32 gates
    (1, 300, 16, torch.bfloat16, False, torch.bfloat16),
    (2, 130, 4, torch.float32, True, torch.bfloat16),
])
def test_dgda_prologue(dev, B, L, H, dtype, with_hist, gdt):
    C = 64 * H
    g = torch.Generator().manual_seed(L * 31 + H)
    xs = [torch.randn(B, L, C, generator=g).to(dtype) for _ in range(6)]
    ws = [torch.randn(C, 1, 4, generator=g) * 0.4 for _ in range(3)]
    hist = [torch.randn(B, C, 3, generator=g).to(dtype) for _ in range(3)] if with_hist else None
    projs = torch.cat(xs, dim=-1).to(dev).split(C, dim=-1)   # views of one GEMM output, row stride 6C
    res = _hip().hip_dgda_prologue(projs, [w.to(dev) for w in ws], [h.to(dev) for h in hist] if hist else None,
                                   n_heads=H, eps=1e-6, gate_dtype=gdt)
    exp = od.layer_prologue(*[to_np(x) for x in xs], *[to_np(w[:, 0]) for w in ws],
                            hist=[to_np(h) for h in hist] if hist else None, n_heads=H, eps=1e-6)
    tol = lambda t: (1e-5, 1e-6) if t.dtype == torch.float32 else (5e-3, 1e-6)  # noqa: E731
    names = ("q", "k", "v", "log_alpha", "alpha", "b", "w")
    for j, name in enumerate(names):
        assert res[j].dtype == (dtype if j < 3 else gdt), name
        assert_close(res[j], exp[j], *tol(res[j]), name)
    for i in range(3):
        assert torch.equal(res[7][i].cpu(), torch.from_numpy(exp[7][i]).to(res[7][i].dtype)), f"history {i}"


def test_dgda_prologue_no_alpha_and_continuation(dev):
    """alpha may be skipped; a prefill cut in two with the history carried equals one pass."""
    B, L, H = 2, 100, 10
    C = 64 * H
    g = torch.Generator().manual_seed(77)
    xs = [torch.randn(B, L, C, generator=g).to(dev) for _ in range(6)]
    ws = [(torch.randn(C, 1, 4, generator=g) * 0.4).to(dev) for _ in range(3)]
    full = _hip().hip_dgda_prologue(xs, ws, None, n_heads=H)
    a = _hip().hip_dgda_prologue([x[:, :45] for x in xs], ws, None, n_heads=H, with_alpha=False)
    b = _hip().hip_dgda_prologue([x[:, 45:] for x in xs], ws, a[7], n_heads=H, with_alpha=False)
    assert a[4] is None and b[4] is None
    for j in (0, 1, 2, 3, 5, 6):
        assert torch.equal(torch.cat([a[j], b[j]], dim=1), full[j]), j
    for i in range(3):
        assert torch.equal(b[7][i], full[7][i])


def test_dgda_prologue_empty_and_fp32_history(dev):
    """L = 0 returns empty outputs and carries the history over unchanged; an fp32 history
    with bf16 projections is read in its own dtype."""
    B, H = 2, 2
    C = 64 * H
    g = torch.Generator().manual_seed(5)
    ws = [(torch.randn(C, 1, 4, generator=g) * 0.4).to(dev) for _ in range(3)]
    hist = [torch.randn(B, C, 3, generator=g).to(dev) for _ in range(3)]
    xs0 = [torch.empty(B, 0, C, device=dev, dtype=torch.bfloat16) for _ in range(6)]
    res = _hip().hip_dgda_prologue(xs0, ws, hist, n_heads=H)
    assert res[0].shape == (B, 0, C)
    for i in range(3):
        assert torch.equal(res[7][i], hist[i])
    xs = [torch.randn(B, 5, C, generator=g).bfloat16() for _ in range(6)]
    res = _hip().hip_dgda_prologue([x.to(dev) for x in xs], ws, hist, n_heads=H, gate_dtype=torch.float32)
    exp = od.layer_prologue(*[to_np(x) for x in xs], *[to_np(w[:, 0]) for w in ws], hist=[to_np(h) for h in hist],
                            n_heads=H)
    assert_close(res[0], exp[0], 5e-3, 1e-6, "q")
    assert_close(res[3], exp[3], 1e-5, 1e-6, "log_alpha")
    for i in range(3):
        assert torch.equal(res[7][i].cpu(), torch.from_numpy(exp[7][i]).float()), i
