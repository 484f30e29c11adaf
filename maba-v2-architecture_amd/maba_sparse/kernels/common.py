"""Input contracts and the PyTorch reference backend of the kernel ops.

These mirror ``maba_sparse/kernels/common.py`` of the reference (validators
``:13-226``, reference ops ``:229-438``) so that the dispatcher's documented
fallback target and its error conventions stay the same: ``ValueError`` for
shapes, ``TypeError`` for dtypes, ``RuntimeError`` for devices.  They are plain
device-agnostic torch code; the HIP kernels never call them.
"""
from __future__ import annotations

import math
from typing import Any, Optional, Tuple, Union

import torch
import torch.nn.functional as F

_FLOAT_DTYPES = (torch.float32, torch.float16, torch.bfloat16, torch.float64)


def normalize_keys(k: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``k / (||k||_2 + eps)`` along the last axis (reference common.py:8-10)."""
    return k / (torch.linalg.vector_norm(k, dim=-1, keepdim=True) + eps)


def _same_device(ref_dev, named) -> None:
    for name, t in named:
        if t is not None and t.device != ref_dev:
            raise RuntimeError(
                f"Expected all tensors to be on the same device, but got {ref_dev} and {t.device} for {name}"
            )


def _same_dtype(ref_dt, named) -> None:
    if ref_dt not in _FLOAT_DTYPES:
        raise TypeError(f"Unsupported dtype {ref_dt}. Supported: {_FLOAT_DTYPES}")
    for name, t in named:
        if t is not None and t.dtype != ref_dt:
            raise TypeError(f"Tensor dtypes must match, but got {ref_dt} for q and {t.dtype} for {name}")


def _gate_tensors(k, v, b, w, alpha, log_alpha):
    named = [("k", k), ("v", v), ("b", b), ("w", w)]
    if alpha is not None:
        named.append(("alpha", alpha))
    if log_alpha is not None:
        named.append(("log_alpha", log_alpha))
    return named


def validate_dgda_prefill_inputs(q, k, v, alpha=None, b=None, w=None, initial_state=None,
                                 check_finite: bool = False, log_alpha=None,
                                 allow_mixed_dtypes: bool = False) -> None:
    """Contract of ``dgda_prefill`` (reference common.py:13-90).

    ``allow_mixed_dtypes`` relaxes the all-tensors-share-q's-dtype rule for the
    HIP backend's mixed-precision mode (bf16 q/k/v with fp32 gates and state).
    """
    if alpha is None and log_alpha is None:
        raise ValueError("Either alpha or log_alpha must be provided")
    if b is None or w is None:
        raise ValueError("Both b and w gate tensors must be provided")
    named = _gate_tensors(k, v, b, w, alpha, log_alpha)
    _same_device(q.device, named + [("initial_state", initial_state)])
    if allow_mixed_dtypes:
        for name, t in [("q", q)] + named + [("initial_state", initial_state)]:
            if t is not None and t.dtype not in _FLOAT_DTYPES:
                raise TypeError(f"Unsupported dtype {t.dtype} for {name}. Supported: {_FLOAT_DTYPES}")
    else:
        _same_dtype(q.dtype, named + [("initial_state", initial_state)])
    if q.dim() != 4:
        raise ValueError(f"q must be 4D [B, H, L, dk], got shape {list(q.shape)}")
    B, H, L, dk = q.shape
    if tuple(k.shape) != (B, H, L, dk):
        raise ValueError(f"k shape {list(k.shape)} must match q shape {(B, H, L, dk)}")
    if v.dim() != 4 or tuple(v.shape[:3]) != (B, H, L):
        raise ValueError(f"v shape {list(v.shape)} must have first 3 dims {(B, H, L)}")
    dv = v.shape[3]
    for name, t, last in (("alpha", alpha, dk), ("log_alpha", log_alpha, dk), ("b", b, dk), ("w", w, dv)):
        if t is not None and tuple(t.shape) != (B, H, L, last):
            raise ValueError(f"{name} shape {list(t.shape)} must match {(B, H, L, last)}")
    if initial_state is not None and tuple(initial_state.shape) != (B, H, dk, dv):
        raise ValueError(f"initial_state shape {list(initial_state.shape)} must match {(B, H, dk, dv)}")
    if check_finite:
        for name, t in [("q", q)] + named:
            if not torch.isfinite(t).all():
                raise ValueError(f"Tensor {name} contains non-finite values (NaN or Inf)")


def validate_dgda_step_inputs(q, k, v, alpha=None, b=None, w=None, state=None,
                              check_finite: bool = False, log_alpha=None,
                              allow_mixed_dtypes: bool = False) -> None:
    """Contract of ``dgda_step`` (reference common.py:93-157)."""
    if alpha is None and log_alpha is None:
        raise ValueError("Either alpha or log_alpha must be provided")
    if b is None or w is None:
        raise ValueError("Both b and w gate tensors must be provided")
    named = _gate_tensors(k, v, b, w, alpha, log_alpha)
    _same_device(q.device, named + [("state", state)])
    if allow_mixed_dtypes:
        for name, t in [("q", q)] + named + [("state", state)]:
            if t is not None and t.dtype not in _FLOAT_DTYPES:
                raise TypeError(f"Unsupported dtype {t.dtype} for {name}. Supported: {_FLOAT_DTYPES}")
    else:
        _same_dtype(q.dtype, named + [("state", state)])
    q3 = q.squeeze(2) if (q.dim() == 4 and q.shape[2] == 1) else q
    if q3.dim() != 3:
        raise ValueError(f"q must be [B, H, dk] or [B, H, 1, dk], got {list(q.shape)}")
    B, H, dk = q3.shape
    v3 = v.squeeze(2) if (v.dim() == 4 and v.shape[2] == 1) else v
    if v3.dim() != 3 or tuple(v3.shape[:2]) != (B, H):
        raise ValueError(f"v must be [B, H, dv] matching B={B}, H={H}, got {list(v.shape)}")
    dv = v3.shape[-1]
    if state is not None and tuple(state.shape) != (B, H, dk, dv):
        raise ValueError(f"state shape {list(state.shape)} must match {(B, H, dk, dv)}")
    if check_finite:
        for name, t in [("q", q)] + named:
            if not torch.isfinite(t).all():
                raise ValueError(f"Tensor {name} contains non-finite values")


def validate_indexer_inputs(k_idx, q_idx=None, centroids=None, check_finite: bool = False) -> None:
    """Contract of the indexer ops (reference common.py:160-192)."""
    if k_idx.dim() != 3:
        raise ValueError(f"k_idx must be 3D [B, L, d_idx], got shape {list(k_idx.shape)}")
    B, L, d_idx = k_idx.shape
    for name, t in (("q_idx", q_idx), ("centroids", centroids)):
        if t is None:
            continue
        if t.device != k_idx.device:
            raise RuntimeError("Expected all tensors to be on the same device")
        if t.dim() != 3 or t.shape[0] != B or t.shape[2] != d_idx:
            raise ValueError(f"{name} shape {list(t.shape)} incompatible with k_idx {(B, L, d_idx)}")
    if check_finite:
        for name, t in (("k_idx", k_idx), ("q_idx", q_idx), ("centroids", centroids)):
            if t is not None and not torch.isfinite(t).all():
                raise ValueError(f"{name} contains non-finite values")


def validate_superposition_inputs(o_local, o_sparse, o_hca, gate_logits_or_weights=None,
                                  check_finite: bool = False) -> None:
    """Contract of ``stream_superposition`` (reference common.py:195-226)."""
    dev = o_local.device
    if o_sparse.device != dev or o_hca.device != dev:
        raise RuntimeError("Expected all tensors to be on the same device")
    if o_local.shape != o_sparse.shape or o_local.shape != o_hca.shape:
        raise ValueError(
            f"Shape mismatch: o_local={list(o_local.shape)}, o_sparse={list(o_sparse.shape)}, "
            f"o_hca={list(o_hca.shape)}"
        )
    g = gate_logits_or_weights
    if g is not None:
        if g.device != dev:
            raise RuntimeError("Expected all tensors to be on the same device")
        if g.shape[-1] != 3:
            raise ValueError(f"Gate tensor last dimension must be 3, got {g.shape[-1]}")
        if g.shape[0] != o_local.shape[0]:
            raise ValueError(f"Gate tensor batch size must match {o_local.shape[0]}")
    if check_finite:
        for name, t in (("o_local", o_local), ("o_sparse", o_sparse), ("o_hca", o_hca)):
            if not torch.isfinite(t).all():
                raise ValueError(f"Tensor {name} contains non-finite values")


# --------------------------------------------------------------------------- reference ops


def ref_dgda_prefill(q, k, v, alpha=None, b=None, w=None, chunk_size: int = 16,
                     initial_state=None, log_alpha=None, **kwargs: Any) -> Tuple[torch.Tensor, torch.Tensor]:
    """Token-sequential DGDA prefill (reference common.py:229-268)."""
    validate_dgda_prefill_inputs(q, k, v, alpha, b, w, initial_state, log_alpha=log_alpha)
    if alpha is None:
        alpha = torch.exp(log_alpha)
    B, H, L, dk = q.shape
    dv = v.shape[-1]
    S = torch.zeros(B, H, dk, dv, dtype=q.dtype, device=q.device) if initial_state is None \
        else initial_state.clone()
    if L == 0:
        return torch.empty(B, H, 0, dv, dtype=q.dtype, device=q.device), S
    outs = []
    for t in range(L):
        Sd = alpha[:, :, t].unsqueeze(-1) * S
        pred = torch.matmul((b[:, :, t] * k[:, :, t]).unsqueeze(-2), Sd)
        delta = (w[:, :, t] * v[:, :, t]).unsqueeze(-2) - pred
        S = Sd + torch.matmul(k[:, :, t].unsqueeze(-1), delta)
        outs.append(torch.matmul(q[:, :, t].unsqueeze(-2), S).squeeze(-2))
    return torch.stack(outs, dim=2), S


def ref_dgda_step(q, k, v, alpha=None, b=None, w=None, state=None, log_alpha=None,
                  **kwargs: Any) -> Tuple[torch.Tensor, torch.Tensor]:
    """One DGDA token (reference common.py:271-309)."""
    validate_dgda_step_inputs(q, k, v, alpha, b, w, state, log_alpha=log_alpha)
    if alpha is None:
        alpha = torch.exp(log_alpha)
    if q.dim() == 4 and q.shape[2] == 1:
        q, k, v, alpha, b, w = (t.squeeze(2) for t in (q, k, v, alpha, b, w))
    B, H, dk = q.shape
    dv = v.shape[-1]
    S = torch.zeros(B, H, dk, dv, dtype=q.dtype, device=q.device) if state is None else state.clone()
    Sd = alpha.unsqueeze(-1) * S
    pred = torch.matmul((b * k).unsqueeze(-2), Sd)
    new_state = Sd + torch.matmul(k.unsqueeze(-1), (w * v).unsqueeze(-2) - pred)
    return torch.matmul(q.unsqueeze(-2), new_state).squeeze(-2), new_state


def ref_dgda_sequential(q, k, v, alpha=None, b=None, w=None, initial_state=None, log_alpha=None,
                        **kwargs: Any):
    return ref_dgda_prefill(q=q, k=k, v=v, alpha=alpha, b=b, w=w, chunk_size=16,
                            initial_state=initial_state, log_alpha=log_alpha, **kwargs)


def ref_compute_centroids(k_idx, block_size: int = 64, **kwargs: Any) -> torch.Tensor:
    """``0.5*(mean+max)`` over zero-padded blocks, in fp32, returned in the input dtype
    (reference common.py:329-350, cpu_indexer.py:38-50)."""
    if k_idx.dim() != 3:
        raise ValueError(f"k_idx must be 3D [B, L, d_idx], got {list(k_idx.shape)}")
    if block_size <= 0:
        raise ValueError(f"block_size must be positive, got {block_size}")
    B, L, d = k_idx.shape
    if d <= 0:
        raise ValueError(f"d_idx must be positive, got {d}")
    if L == 0:
        return torch.empty(B, 0, d, dtype=k_idx.dtype, device=k_idx.device)
    kf = k_idx.float() if k_idx.dtype in (torch.float16, torch.bfloat16) else k_idx
    nb = (L + block_size - 1) // block_size
    pad = nb * block_size - L
    kp = F.pad(kf, (0, 0, 0, pad)) if pad else kf
    kb = kp.reshape(B, nb, block_size, d)
    return (0.5 * (kb.mean(dim=2) + kb.amax(dim=2))).to(k_idx.dtype)


def ref_index_topk(q_idx, centroids, lambda_dist: float = 0.5, top_k: int = 32, block_size: int = 64,
                   return_scores: bool = False, **kwargs: Any):
    """Causal prefill scoring + top-k in fp32 (reference cpu_indexer.py:53-112)."""
    lam = kwargs.get("dist_lambda", lambda_dist)
    if q_idx.device != centroids.device:
        raise RuntimeError(
            f"Expected all tensors to be on the same device, got {q_idx.device} and {centroids.device}")
    if q_idx.dim() != 3 or centroids.dim() != 3:
        raise ValueError(f"q_idx and centroids must be 3D, got {q_idx.dim()}D and {centroids.dim()}D")
    if top_k <= 0:
        raise ValueError(f"top_k must be positive, got {top_k}")
    if block_size <= 0:
        raise ValueError(f"block_size must be positive, got {block_size}")
    B, L, d = q_idx.shape
    nb = centroids.shape[1]
    ak = min(top_k, nb)
    if L == 0 or nb == 0:
        idx = torch.zeros(B, L, ak, dtype=torch.long, device=q_idx.device)
        if return_scores:
            return idx, torch.zeros(B, L, nb, dtype=q_idx.dtype, device=q_idx.device)
        return idx
    s = torch.bmm(q_idx.float() * (1.0 / math.sqrt(d)), centroids.float().transpose(1, 2))
    qi = torch.arange(L, device=q_idx.device).unsqueeze(1) // block_size
    ni = torch.arange(nb, device=q_idx.device).unsqueeze(0)
    sc = s - (lam * torch.log1p((qi - ni).abs().float())).unsqueeze(0)
    sc = sc.masked_fill((ni > qi).unsqueeze(0), float("-inf"))
    idx = torch.topk(sc, k=ak, dim=-1, largest=True, sorted=True).indices.to(torch.long)
    if return_scores:
        return idx, sc.to(q_idx.dtype)
    return idx


def ref_index_topk_decode(q, centroids, lambda_dist: float = 0.5, top_k: int = 32,
                          return_scores: bool = False, **kwargs: Any):
    """Decode scoring (query block = nb-1, no mask) + top-k for ``q [B, Hq, d]``
    (reference layers/indexer.py:101-112, computed in fp32)."""
    lam = kwargs.get("dist_lambda", lambda_dist)
    nb = centroids.shape[1]
    d = q.shape[-1]
    dot = torch.matmul(q.float() * (1.0 / math.sqrt(d)), centroids.float().transpose(-1, -2))
    dist = (nb - 1 - torch.arange(nb, device=q.device)).clamp(min=0).float()
    scores = dot - (lam * torch.log1p(dist)).view(1, 1, nb)
    idx = torch.topk(scores, k=min(top_k, nb), dim=-1, largest=True, sorted=True).indices
    if return_scores:
        return idx, scores
    return idx


def ref_stream_superposition(o_local, o_sparse, o_hca, gate_logits=None, gate_weights=None,
                             **kwargs: Any) -> torch.Tensor:
    """``g0*o_local + g1*o_sparse + g2*o_hca`` (reference common.py:406-438)."""
    gate = gate_logits if gate_logits is not None else gate_weights
    validate_superposition_inputs(o_local, o_sparse, o_hca, gate)
    if o_local.shape[2] == 0:
        return torch.empty_like(o_local)
    if gate_weights is None:
        if gate_logits is None:
            raise ValueError("Either gate_logits or gate_weights must be provided")
        g = F.softmax(gate_logits.float(), dim=-1).to(o_local.dtype)
    else:
        g = gate_weights.to(o_local.dtype)
    if g.dim() == 3:
        g = g.unsqueeze(1)
    elif g.dim() != 4:
        raise ValueError(f"Gate tensor must be 3D or 4D, got {g.dim()}D")
    return g[..., 0:1] * o_local + g[..., 1:2] * o_sparse + g[..., 2:3] * o_hca


def ref_hca_pool(c_kv, pool: int = 64, **kwargs: Any) -> torch.Tensor:
    """Means of complete ``pool``-token blocks (reference layers/sparse_attention.py:206)."""
    B, L, dc = c_kv.shape
    nc = L // pool
    return c_kv[:, : nc * pool].float().reshape(B, nc, pool, dc).mean(dim=2).to(c_kv.dtype)


def ref_maba_sa_decode(q_lat, c_kv, hca, idx, gate, L: int, scale: float, window: int = 128,
                       n_sink: int = 4, block_size: int = 64, pool: int = 64, **kwargs: Any) -> torch.Tensor:
    """Latent-space MABA-SA decode step (reference layers/sparse_attention.py:79-219,263-275).

    Returns ``sum_s g_s * sum_j p_sj c_j`` of shape ``[B, H, dc]`` in fp32; the
    caller applies the per-head value up-projection.
    """
    B, H, dc = q_lat.shape
    q = q_lat.float() * scale
    c = c_kv[:, :L].float()
    dev = q.device
    ns = min(n_sink, L)
    loc = torch.cat([torch.arange(ns, device=dev), torch.arange(max(ns, L - window), L, device=dev)])

    def attend(keys: torch.Tensor, valid: Optional[torch.Tensor] = None) -> torch.Tensor:
        s = torch.einsum("bhd,bnd->bhn", q, keys)
        if valid is not None:
            s = s.masked_fill(~valid, float("-inf"))
        p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
        return torch.einsum("bhn,bnd->bhd", p, keys)

    z_loc = attend(c[:, loc])
    z_sp = torch.zeros(B, H, dc, device=dev)
    offs = torch.arange(block_size, device=dev)
    for b in range(B):
        for h in range(H):
            row = idx[b, 0] if idx.shape[1] == 1 else idx[b, h]
            pos = (row.view(-1, 1) * block_size + offs.view(1, -1)).reshape(-1)
            pos = pos[(pos < L) & (pos >= 0)]
            keys = c[b, pos]
            s = keys @ q[b, h]
            z_sp[b, h] = torch.softmax(s, dim=0) @ keys if pos.numel() else 0.0
    if L - 1 < pool - 1:
        z_hca = c.mean(dim=1, keepdim=True).expand(B, H, dc)
    else:
        z_hca = attend(hca[:, : L // pool].float())
    g = torch.softmax(gate.float(), dim=-1)
    g = g.view(B, 1, 3) if g.dim() == 2 else g
    return g[..., 0:1] * z_loc + g[..., 1:2] * z_sp + g[..., 2:3] * z_hca


def ref_maba_sa_prefill(q, k, v, kh, vh, early, idx, gate_logits, scale: float, window: int = 128,
                        n_sink: int = 4, block_size: int = 64, pool: int = 64, out_dtype=None, **kwargs: Any):
    """MABA-SA prefill streams and their gate (reference layers/sparse_attention.py:95-105,
    145-171, 173-219, 275) with dense masks, in fp32.

    q ``[B,H,Lq,dh]``, k/v ``[B,H,Lkv,dh]`` per-head keys and values, kh/vh ``[B,H,Lkv//pool,dh]``
    the up-projected complete-block means, early ``[B,H,n_early,dh]`` the rows of the queries
    before position ``pool - 1`` (or None), idx ``[B,Lq|1,K]``, gate logits ``[B,Lq,3]`` or
    ``[B,H,Lq,3]``.  A block listed twice in a row counts twice.  Returns ``[B,H,Lq,dh]``
    (computed in fp32, or fp64 for fp64 inputs)."""
    B, H, Lq, dh = q.shape
    Lkv = k.shape[2]
    dev = q.device
    ct = torch.promote_types(q.dtype, torch.float32)
    qf, kf, vf = q.to(ct), k.to(ct), v.to(ct)
    pos = (Lkv - Lq) + torch.arange(Lq, device=dev)
    j = torch.arange(Lkv, device=dev)
    ns = min(n_sink, Lkv)

    def attend(s, w, vals):
        s = s.masked_fill(w <= 0, float("-inf"))
        m = s.amax(dim=-1, keepdim=True)
        m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
        p = w * torch.exp(s - m)
        tot = p.sum(dim=-1, keepdim=True)
        return torch.where(tot > 0, (p / tot.clamp_min(1e-38)) @ vals, torch.zeros((), device=dev))

    s = (qf @ kf.transpose(-1, -2)) * scale                                  # [B,H,Lq,Lkv]
    local_w = ((j[None] <= pos[:, None]) & (((pos[:, None] - j[None]) < window) | (j[None] < ns))).to(ct)
    ol = attend(s, local_w[None, None], vf)
    nb = (Lkv + block_size - 1) // block_size
    rows = idx if idx.shape[1] == Lq else idx[:, :1].expand(B, Lq, idx.shape[2])
    blk_of = (j // block_size)[None, None, None, :]                         # [1,1,1,Lkv]
    ok = (rows >= 0) & (rows < nb)
    cnt = ((rows[..., None] == blk_of) & ok[..., None]).sum(dim=2).to(ct)   # [B,Lq,Lkv]
    sp_w = cnt * (j[None, None] <= pos[None, :, None]).to(ct)
    os_ = attend(s, sp_w[:, None], vf)
    nc = Lkv // pool
    oh = torch.zeros_like(ol)
    if nc > 0:
        ends = (torch.arange(nc, device=dev) + 1) * pool - 1
        hca_w = (ends[None] <= pos[:, None]).to(ct)
        oh = attend((qf @ kh.to(ct).transpose(-1, -2)) * scale, hca_w[None, None], vh.to(ct))
    n_early = int((pos < pool - 1).sum())
    if n_early > 0:
        oh[:, :, :n_early] = early[:, :, :n_early].to(ct)
    g = torch.softmax(gate_logits.to(ct), dim=-1)
    g = g[:, None] if g.dim() == 3 else g
    out = g[..., 0:1] * ol + g[..., 1:2] * os_ + g[..., 2:3] * oh
    return out.to(out_dtype or q.dtype)


def ref_dgda_prologue(projections, conv_weights, history=None, n_heads: int = 10, eps: float = 1e-6,
                      gate_dtype: Optional[torch.dtype] = None, with_alpha: bool = True, **kwargs: Any):
    """DGDA layer prologue (reference layers/dgda.py:103-121, 186-207) in torch.

    ``projections`` = (x_q, x_k, x_v, x_alpha, x_erase, x_write), each ``[B, L, C]``;
    ``conv_weights`` = three depthwise ``[C, 1, K]`` kernels; ``history`` = three
    ``[B, C, K-1]`` carried conv inputs or None.  Returns ``(q, k, v, log_alpha, alpha,
    b, w, (hq, hk, hv))`` with q/k/v ``[B, L, C]`` in the projections' dtype and the gates in
    ``gate_dtype`` (default: that dtype); k is normalised per ``C // n_heads``-channel head.
    """
    xq, xk, xv, xa, xb, xw = projections
    B, L, C = xq.shape
    dt = xq.dtype
    outs, hists = [], []
    for i, (x, wgt) in enumerate(zip((xq, xk, xv), conv_weights)):
        kh = wgt.shape[-1] - 1
        xt = x.transpose(1, 2)
        hist = None if history is None else history[i]
        seq = F.pad(xt, (kh, 0)) if hist is None else torch.cat([hist.to(dt), xt], dim=2)
        hists.append(seq[..., seq.shape[-1] - kh:].contiguous())
        outs.append(F.silu(F.conv1d(seq, wgt.to(dt), groups=C)).transpose(1, 2))
    q, k, v = outs
    dk = C // n_heads
    kh_ = k.reshape(B, L, n_heads, dk)
    k = (kh_ / (torch.linalg.vector_norm(kh_, dim=-1, keepdim=True) + eps)).reshape(B, L, C)
    gdt = gate_dtype or dt
    la = torch.clamp(-F.softplus(xa), min=-14.0)
    alpha = torch.exp(la).to(gdt) if with_alpha else None
    return (q, k, v, la.to(gdt), alpha, torch.sigmoid(xb).to(gdt), torch.sigmoid(xw).to(gdt), tuple(hists))


reference_dgda_prefill = ref_dgda_prefill
reference_dgda_step = ref_dgda_step
reference_dgda_sequential = ref_dgda_sequential
reference_compute_centroids = ref_compute_centroids
reference_index_topk = ref_index_topk
reference_stream_superposition = ref_stream_superposition
ref_centroids = ref_compute_centroids
ref_topk = ref_index_topk
ref_superposition = ref_stream_superposition
