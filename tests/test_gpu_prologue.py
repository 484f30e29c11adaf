"""The DGDA layer prologue kernel (conv + SiLU with carried history, gates, key norm)
against the float64 oracle (``oracle.dgda.layer_prologue``) on seeded inputs, and the
layer prefill with the prologue fused into the recurrence kernels against the float64
prologue composed with the float64 token recurrence (``oracle.dgda.dgda_prefill_seq``).

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


# ---------------------------------------------------------------- the fused layer prefill

def _fused_case(B, L, H, seed, with_hist, with_state, slow):
    C = 64 * H
    g = torch.Generator().manual_seed(seed)
    xs = [torch.randn(B, L, C, generator=g).bfloat16() for _ in range(6)]
    if slow:   # decay projections far below zero: log alpha ~ -e^{x}, a long memory
        xs[3] = (torch.randn(B, L, C, generator=g) - 6.0).bfloat16()
    ws = [torch.randn(C, 1, 4, generator=g) * 0.4 for _ in range(3)]
    hist = [torch.randn(B, C, 3, generator=g).bfloat16() for _ in range(3)] if with_hist else None
    s0 = torch.randn(B, H, 64, 64, generator=g) * 0.1 if with_state else None
    return xs, ws, hist, s0


def _fused_oracle(xs, ws, hist, s0, H, eps=1e-6):
    """The float64 prologue, then the float64 token recurrence on its outputs."""
    B, L, C = xs[0].shape
    q, k, v, la, _, b, w, nh = od.layer_prologue(*[to_np(x) for x in xs], *[to_np(c[:, 0]) for c in ws],
                                                 hist=[to_np(h) for h in hist] if hist else None, n_heads=H, eps=eps)
    heads = lambda t: t.reshape(B, L, H, 64).transpose(0, 2, 1, 3)  # noqa: E731
    eo, eS = od.dgda_prefill_seq(heads(q), heads(k), heads(v), b=heads(b), w=heads(w),
                                    initial_state=to_np(s0) if s0 is not None else None, log_alpha=heads(la))
    return eo.transpose(0, 2, 1, 3).reshape(B, L, C), eS, nh


@pytest.mark.parametrize("B,L,H,with_hist,with_state,slow", [
    (2, 1, 2, True, True, False),       # one token: its three earlier taps from the history
    (1, 2, 2, True, False, False),      # L < 3: the new history keeps the old one's tail
    (2, 37, 3, False, True, False),     # ragged last sub-chunk, zero history
    (1, 1500, 2, True, True, True),     # slow decay: the state reaches across sub-chunks
    (2, 2500, 10, True, False, False),  # the layer's head count
])
def test_dgda_layer_prefill_fused_vs_oracle(dev, B, L, H, with_hist, with_state, slow):
    """Rtol = atol = 2e-3 on the fp32 outputs and the final state (the north-star DGDA bar,
    bf16 inputs with fp32 accumulation); the new history is a copy of inputs: exact."""
    xs, ws, hist, s0 = _fused_case(B, L, H, L * 13 + H, with_hist, with_state, slow)
    d = lambda t: None if t is None else t.to(dev)  # noqa: E731
    projs = torch.cat(xs, dim=-1).to(dev).split(64 * H, dim=-1)   # views of one GEMM output, row stride 6C
    out = torch.empty(B, L, 64 * H, device=dev)
    o, S, nh = _hip().hip_dgda_layer_prefill(projs, [d(w) for w in ws], [d(h) for h in hist] if hist else None,
                                             eps=1e-6, initial_state=d(s0), out=out, state_dtype=torch.float32)
    eo, eS, enh = _fused_oracle(xs, ws, hist, s0, H)
    assert o.data_ptr() == out.data_ptr()
    assert_close(o, eo, 2e-3, 2e-3, f"out L={L}")
    assert_close(S, eS, 2e-3, 2e-3, f"state L={L}")
    for i in range(3):
        assert torch.equal(nh[i].cpu().float(), torch.from_numpy(enh[i]).float()), f"history {i}"


def test_dgda_layer_prefill_fused_split_and_bf16_out(dev):
    """A prefill cut in two, the state and the conv history carried (the history rewritten in
    place), equals one pass; the bf16 output is the rounding of the fp32 one."""
    B, L, H = 2, 700, 4
    xs, ws, _, _ = _fused_case(B, L, H, 3, False, False, True)
    projs = torch.cat(xs, dim=-1).to(dev).split(64 * H, dim=-1)
    wd = [w.to(dev) for w in ws]
    hb = _hip()
    out = torch.empty(B, L, 64 * H, device=dev)
    o, S, nh = hb.hip_dgda_layer_prefill(projs, wd, None, out=out, state_dtype=torch.float32)
    cut = 301
    o1, S1, nh1 = hb.hip_dgda_layer_prefill([p[:, :cut] for p in projs], wd, None, state_dtype=torch.float32,
                                            out=torch.empty(B, cut, 64 * H, device=dev))
    o2, S2, nh2 = hb.hip_dgda_layer_prefill([p[:, cut:] for p in projs], wd, nh1, initial_state=S1,
                                            out_history=nh1, state_dtype=torch.float32,
                                            out=torch.empty(B, L - cut, 64 * H, device=dev))
    assert nh2[0].data_ptr() == nh1[0].data_ptr()
    assert_close(torch.cat([o1, o2], dim=1), to_np(o), 2e-3, 2e-3, "split outputs")
    assert_close(S2, to_np(S), 2e-3, 2e-3, "split state")
    for i in range(3):
        assert torch.equal(nh2[i], nh[i])
    obf, _, _ = hb.hip_dgda_layer_prefill(projs, wd, None)
    assert obf.dtype == torch.bfloat16
    assert torch.equal(obf, o.bfloat16())


def test_dgda_layer_fused_forward_matches_unfused(dev):
    """The bf16 DGDALayer with the prologue fused against the same layer with the one-pass
    prologue kernel and the op on its stored bf16 outputs (which round q, k, v once more):
    within 2e-2 of the output's largest magnitude; then a second call continues from the
    returned state and conv history in both."""
    from maba_sparse.layers import DGDALayer
    torch.manual_seed(2)
    layer = DGDALayer(dim=256, n_heads=4).to(dev, torch.bfloat16).eval()
    x = torch.randn(2, 900, 256, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        yf, sf, cf = layer(x[:, :500])
        yf2, sf2, _ = layer(x[:, 500:], state=sf, conv_state=cf)
        layer.fuse_prologue = False
        yu, su, cu = layer(x[:, :500])
        yu2, su2, _ = layer(x[:, 500:], state=su, conv_state=cu)
    for a, b_, name in ((yf, yu, "y"), (yf2, yu2, "y2"), (sf, su, "S"), (sf2, su2, "S2")):
        err = (a.float() - b_.float()).abs().max().item()
        assert err <= 2e-2 * b_.float().abs().max().item(), (name, err)
    for i in range(3):
        assert torch.equal(cf[i], cu[i]), f"history {i}"


@pytest.mark.parametrize("B,H,sdt,with_hist", [
    (16, 10, torch.bfloat16, True),    # the serving model's decode shape and state dtype
    (3, 4, torch.float32, True),
    (2, 16, torch.bfloat16, False),    # no history: zero taps
])
def test_dgda_layer_step_equals_prologue_then_step(dev, B, H, sdt, with_hist):
    """The one-launch decode token (prologue + step) against the two launches it replaces,
    which the tests above and the decode tests pin to the oracle: equal bit for bit (the
    same arithmetic, q/k/v rounded to bf16 and the gates kept in fp32 in both), the state
    and the conv history updated in place."""
    hb = _hip()
    C = 64 * H
    g = torch.Generator().manual_seed(B * 100 + H)
    proj = torch.randn(B, 1, 6 * C, generator=g).to(dev, torch.bfloat16)
    projs = proj.split(C, dim=-1)
    ws = [(torch.randn(C, 1, 4, generator=g) * 0.4).to(dev) for _ in range(3)]
    hist = [torch.randn(B, C, 3, generator=g).to(dev, torch.bfloat16) for _ in range(3)] if with_hist else None
    state = (torch.randn(B, H, 64, 64, generator=g) * 0.3).to(dev, sdt)
    # two launches
    h1 = [h.clone() for h in hist] if with_hist else [torch.empty(B, C, 3, device=dev, dtype=torch.bfloat16)
                                                      for _ in range(3)]
    s1 = state.clone()
    q, k, v, la, _, b, w, _ = hb.hip_dgda_prologue(projs, ws, tuple(h1) if with_hist else None, n_heads=H, eps=1e-6,
                                                   gate_dtype=torch.float32, with_alpha=False, out_history=tuple(h1))
    o1, _ = hb.hip_dgda_step(q.view(B, H, 64), k.view(B, H, 64), v.view(B, H, 64), log_alpha=la.view(B, H, 64),
                             b=b.view(B, H, 64), w=w.view(B, H, 64), state=s1, new_state=s1, allow_mixed_dtypes=True)
    # one launch
    h2 = [h.clone() for h in hist] if with_hist else [torch.zeros(B, C, 3, device=dev, dtype=torch.bfloat16)
                                                      for _ in range(3)]
    s2 = state.clone()
    o2 = hb.hip_dgda_layer_step(projs, ws, tuple(h2), s2, eps=1e-6)
    assert o2.dtype == o1.dtype and o2.shape == (B, H, 64)
    assert torch.equal(o2, o1.view(B, H, 64)), "o"
    assert torch.equal(s2, s1), "state"
    for i in range(3):
        assert torch.equal(h2[i], h1[i]), f"history {i}"


def test_dgda_layer_step_device_fused_matches_unfused(dev):
    """DGDALayer.step_device (the serving path) with the fused launch against the same layer
    with the prologue and the step as two launches, over two consecutive tokens."""
    from maba_sparse.layers import DGDALayer
    torch.manual_seed(4)
    layer = DGDALayer(dim=640, n_heads=10).to(dev, torch.bfloat16).eval()
    B, C = 16, 640
    st = (torch.randn(B, 10, 64, 64, device=dev) * 0.2).to(torch.bfloat16)
    hs = [torch.randn(B, C, 3, device=dev).to(torch.bfloat16) for _ in range(3)]
    xs = [torch.randn(B, 1, C, device=dev, dtype=torch.bfloat16) for _ in range(2)]
    outs = {}
    for fused in (True, False):
        layer.fuse_prologue = fused
        s, h = st.clone(), [x.clone() for x in hs]
        with torch.no_grad():
            outs[fused] = [layer.step_device(x, s, h) for x in xs] + [s, *h]
    for a, b_ in zip(outs[True], outs[False]):
        assert torch.equal(a, b_)
