"""Seeded input builders and comparison helpers shared by the tests."""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def dgda_inputs(B, H, L, dk=64, dv=64, qkv_dtype=torch.bfloat16, gate_dtype=torch.float32,
                gates="scalar", decay="baseline", seed=0, device="cpu", with_state=False):
    """Synthetic DGDA inputs with the BASELINE distributions.

    q, k ~ N(0,1) L2-normalised per head; v ~ N(0,1); beta = sigmoid(N(0,1)) used
    for both b and w; log-decay = -softplus(N(0,1)+2) ("baseline"), a slow decay
    ("slow", ~0.5% per token) or none ("none").  ``gates="scalar"`` gives one
    value per token broadcast over channels with a stride-0 view;
    ``gates="channel"`` draws every channel independently.
    """
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, L, dk, generator=g)
    k = torch.randn(B, H, L, dk, generator=g)
    q = q / q.norm(dim=-1, keepdim=True).clamp_min(1e-6)
    k = k / k.norm(dim=-1, keepdim=True).clamp_min(1e-6)
    v = torch.randn(B, H, L, dv, generator=g)
    if gates == "scalar":
        z_a = torch.randn(B, H, L, 1, generator=g)
        z_b = torch.randn(B, H, L, 1, generator=g)
    else:
        z_a = torch.randn(B, H, L, dk, generator=g)
        z_b = torch.randn(B, H, L, max(dk, dv), generator=g)
    if decay == "baseline":
        la = -F.softplus(z_a + 2.0)
    elif decay == "slow":
        la = -F.softplus(z_a + 2.0) * 0.005
    elif decay == "none":
        la = torch.zeros_like(z_a)
    else:
        raise ValueError(decay)
    beta = torch.sigmoid(z_b)
    s0 = torch.randn(B, H, dk, dv, generator=g) * 0.1 if with_state else None
    # move to the device before broadcasting: .to(device) would materialise a stride-0 view
    la = la.to(device=device, dtype=gate_dtype)
    beta = beta.to(device=device, dtype=gate_dtype)
    if gates == "scalar":
        la_t = la.expand(B, H, L, dk)
        b_t = beta.expand(B, H, L, dk)
        w_t = beta.expand(B, H, L, dv)
    else:
        la_t = la
        b_t = beta[..., :dk]
        w_t = beta[..., :dv]
    return dict(q=q.to(device=device, dtype=qkv_dtype), k=k.to(device=device, dtype=qkv_dtype),
                v=v.to(device=device, dtype=qkv_dtype), log_alpha=la_t, b=b_t, w=w_t,
                initial_state=None if s0 is None else s0.to(device))


def to_np(t):
    return None if t is None else t.detach().double().cpu().numpy()


def oracle_dgda_args(inp):
    """float64 numpy arguments for ``oracle.dgda.dgda_prefill_seq`` from the exact stored inputs."""
    la = to_np(inp["log_alpha"])
    return dict(q=to_np(inp["q"]), k=to_np(inp["k"]), v=to_np(inp["v"]), alpha=np.exp(la),
                b=to_np(inp["b"]), w=to_np(inp["w"]), initial_state=to_np(inp.get("initial_state")))


def assert_close(actual, expected, rtol, atol, what=""):
    a = actual.detach().double().cpu().numpy() if isinstance(actual, torch.Tensor) else np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape, f"{what}: shape {a.shape} vs {e.shape}"
    bad = np.abs(a - e) > atol + rtol * np.abs(e)
    if bad.any():
        i = np.unravel_index(np.argmax(np.abs(a - e) - rtol * np.abs(e)), a.shape)
        raise AssertionError(
            f"{what}: {bad.sum()} / {bad.size} elements outside rtol={rtol} atol={atol}; "
            f"worst at {i}: got {a[i]!r} expected {e[i]!r} (max abs err {np.abs(a - e).max():.3e})")


def topk_agrees(idx_actual, scores_ref, k, gap=1e-4):
    """Top-k selections agree wherever the reference's scores separate them.

    For each row: the selected *sets* must be equal when the gap between the
    k-th and (k+1)-th reference score exceeds ``gap``, and positions whose
    neighbouring reference scores differ by more than ``gap`` must hold the same
    index.  Returns the number of rows checked exactly.
    """
    ia = np.asarray(idx_actual).reshape(-1, idx_actual.shape[-1])
    s = np.asarray(scores_ref, np.float64).reshape(ia.shape[0], -1)
    n = s.shape[1]
    ak = min(k, n)
    checked = 0
    for r in range(ia.shape[0]):
        order = np.lexsort((np.arange(n), -s[r]))
        ref_sorted = s[r][order]
        with np.errstate(invalid="ignore"):
            sep = ref_sorted[ak - 1] - ref_sorted[ak] if ak < n else np.inf
        if not (sep > gap):  # tied or both -inf: torch.topk leaves the order open
            continue
        checked += 1
        assert set(ia[r].tolist()) == set(order[:ak].tolist()), f"row {r}: selected set differs"
        for p in range(ak):
            with np.errstate(invalid="ignore"):
                lo = ref_sorted[p - 1] - ref_sorted[p] if p > 0 else np.inf
                hi = ref_sorted[p] - ref_sorted[p + 1] if p + 1 < n else np.inf
            if lo > gap and hi > gap:
                assert ia[r][p] == order[p], f"row {r} rank {p}: {ia[r][p]} vs {order[p]}"
    return checked


def topk_is_valid(idx_actual, scores_ref, tol=1e-4):
    """Every row's selection is a top-k of the reference scores up to ``tol``: no unselected
    score exceeds a selected one by more than ``tol``, and no index repeats.  Holds for the
    rows whose k-th gap is too small for ``topk_agrees`` to compare them."""
    ia = np.asarray(idx_actual).reshape(-1, idx_actual.shape[-1])
    s = np.asarray(scores_ref, np.float64).reshape(ia.shape[0], -1)
    for r in range(ia.shape[0]):
        sel = ia[r]
        assert len(set(sel.tolist())) == sel.size, f"row {r}: repeated index"
        mask = np.ones(s.shape[1], bool)
        mask[sel] = False
        if mask.any():
            worst_in, best_out = s[r][sel].min(), s[r][mask].max()
            assert best_out <= worst_in + tol, f"row {r}: unselected {best_out} above selected {worst_in}"
