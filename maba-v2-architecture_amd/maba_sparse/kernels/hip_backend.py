"""The ``"hip"`` backend: registered wrappers around ``libmaba_hip.so``.

Each wrapper keeps the reference op's keyword signature and return
convention, allocates outputs (and any workspace) with torch on the inputs'
device, and enqueues the HIP kernels on torch's current stream; the library
itself never allocates.  The kernels are forward-only: when autograd needs
gradients a wrapper raises ``NotImplementedError`` so that the dispatcher falls
back to the differentiable reference path (reference tests check gradients
through the dispatcher, tests/test_dispatcher.py:324-443).

Reference wrappers mirrored (paths relative to the reference checkout):
``triton_dgda_prefill``/``triton_dgda_step`` (kernels/triton_dgda.py:647-685),
``triton_compute_centroids``/``triton_index_topk``/``triton_stream_superposition``
(kernels/triton_indexer.py:558-693).
"""
from __future__ import annotations

import math
from typing import Any, Optional, Tuple

import torch

from maba_sparse import _native as N
from maba_sparse.kernels.common import (
    validate_dgda_prefill_inputs,
    validate_dgda_step_inputs,
    validate_indexer_inputs,
    validate_superposition_inputs,
)
from maba_sparse.kernels.dispatcher import register_kernel


def _no_grad_needed(op: str, *tensors) -> None:
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        raise NotImplementedError(f"{op}: HIP kernels are forward-only; autograd uses the reference path")


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


@register_kernel("hip", "dgda_prefill")
def hip_dgda_prefill(q, k, v, alpha=None, b=None, w=None, chunk_size: int = 16, initial_state=None,
                     log_alpha=None, out_dtype: Optional[torch.dtype] = None,
                     state_dtype: Optional[torch.dtype] = None, allow_mixed_dtypes: bool = False,
                     **kwargs: Any) -> Tuple[torch.Tensor, torch.Tensor]:
    """Chunked DGDA prefill on gfx950 (reference contract: dispatcher.py:258-327).

    Outputs default to q's dtype like the reference (cpu_dgda.py:197);
    ``out_dtype``/``state_dtype`` override them.  ``inversion_method`` and
    ``adaptive_tol`` are accepted and ignored: the kernel's triangular solves
    are exact.
    """
    validate_dgda_prefill_inputs(q, k, v, alpha, b, w, initial_state, log_alpha=log_alpha,
                                 allow_mixed_dtypes=allow_mixed_dtypes)
    _no_grad_needed("dgda_prefill", q, k, v, alpha, b, w, initial_state, log_alpha)
    dev = N.require_device([q, k, v, alpha, b, w, initial_state, log_alpha], "dgda_prefill")
    B, H, L, dk = q.shape
    dv = v.shape[-1]
    odt = out_dtype or q.dtype
    sdt = state_dtype or q.dtype
    if L == 0:
        st = initial_state.clone().to(sdt) if initial_state is not None else \
            torch.zeros(B, H, dk, dv, dtype=sdt, device=dev)
        return torch.empty(B, H, 0, dv, dtype=odt, device=dev), st
    lib = N.load()
    out = torch.empty(B, H, L, dv, dtype=odt, device=dev)
    state = torch.empty(B, H, dk, dv, dtype=sdt, device=dev)
    dq, dk_, dvv = N.desc(q), N.desc(k), N.desc(v)
    da, dla = N.desc(alpha), N.desc(log_alpha)
    db, dw = N.desc(b), N.desc(w)
    ds0 = N.desc(initial_state)
    dout, dst = N.desc(out), N.desc(state)
    gate = dla if log_alpha is not None else da
    nbytes = lib.maba_hip_dgda_prefill_workspace_size(dq, dvv, gate, db)
    ws = _workspace(nbytes, dev)
    rc = lib.maba_hip_dgda_prefill(dq, dk_, dvv, da, dla, db, dw, ds0, dout, dst, int(chunk_size),
                                   ws.data_ptr(), ws.numel(), N.stream_ptr(dev))
    N.check(rc, "dgda_prefill")
    return out, state


def _squeeze_step(t):
    if t is None:
        return None
    return t.squeeze(2) if (t.dim() == 4 and t.shape[2] == 1) else t


@register_kernel("hip", "dgda_step")
def hip_dgda_step(q, k, v, alpha=None, b=None, w=None, state=None, log_alpha=None,
                  out_dtype: Optional[torch.dtype] = None, state_dtype: Optional[torch.dtype] = None,
                  allow_mixed_dtypes: bool = False, **kwargs: Any) -> Tuple[torch.Tensor, torch.Tensor]:
    """One DGDA decode token (reference contract: dispatcher.py:330-396)."""
    validate_dgda_step_inputs(q, k, v, alpha, b, w, state, log_alpha=log_alpha,
                              allow_mixed_dtypes=allow_mixed_dtypes)
    _no_grad_needed("dgda_step", q, k, v, alpha, b, w, state, log_alpha)
    dev = N.require_device([q, k, v, alpha, b, w, state, log_alpha], "dgda_step")
    q3, k3, v3, a3, b3, w3, la3 = (_squeeze_step(t) for t in (q, k, v, alpha, b, w, log_alpha))
    B, H, dk = q3.shape
    dv = v3.shape[-1]
    out = torch.empty(B, H, dv, dtype=out_dtype or q.dtype, device=dev)
    new_state = kwargs.get("new_state")   # caller buffer; may be `state` itself (updated in place)
    if new_state is None:
        new_state = torch.empty(B, H, dk, dv, dtype=state_dtype or q.dtype, device=dev)
    lib = N.load()
    rc = lib.maba_hip_dgda_step(N.desc(q3), N.desc(k3), N.desc(v3), N.desc(a3), N.desc(la3), N.desc(b3),
                                N.desc(w3), N.desc(state), N.desc(out), N.desc(new_state), N.stream_ptr(dev))
    N.check(rc, "dgda_step")
    return out, new_state


@register_kernel("hip", "compute_centroids")
def hip_compute_centroids(k_idx, block_size: int = 64, **kwargs: Any) -> torch.Tensor:
    """Block centroids (reference contract: dispatcher.py:399-421, triton_indexer.py:558-578)."""
    validate_indexer_inputs(k_idx=k_idx)
    if block_size <= 0:
        raise ValueError(f"block_size must be positive, got {block_size}")
    _no_grad_needed("compute_centroids", k_idx)
    dev = N.require_device([k_idx], "compute_centroids")
    B, L, d = k_idx.shape
    nb = (L + block_size - 1) // block_size
    out = torch.empty(B, nb, d, dtype=k_idx.dtype, device=dev)
    if L == 0:
        return out
    rc = N.load().maba_hip_compute_centroids(N.desc(k_idx), N.desc(out), int(block_size), N.stream_ptr(dev))
    N.check(rc, "compute_centroids")
    return out


@register_kernel("hip", "index_topk")
def hip_index_topk(q_idx, centroids, lambda_dist: float = 0.5, top_k: int = 32, block_size: int = 64,
                   return_scores: bool = False, **kwargs: Any):
    """Causal prefill scoring + top-k (reference contract: dispatcher.py:424-465)."""
    lam = kwargs.get("dist_lambda", lambda_dist)
    if q_idx.device != centroids.device:
        raise RuntimeError(
            f"Expected all tensors to be on the same device, got {q_idx.device} and {centroids.device}")
    if q_idx.dim() != 3 or centroids.dim() != 3:
        raise ValueError(f"q_idx and centroids must be 3D, got {q_idx.dim()}D and {centroids.dim()}D")
    if q_idx.shape[0] != centroids.shape[0] or q_idx.shape[2] != centroids.shape[2]:
        raise ValueError(
            f"Dimension mismatch between q_idx {list(q_idx.shape)} and centroids {list(centroids.shape)}")
    if top_k <= 0:
        raise ValueError(f"top_k must be positive, got {top_k}")
    if block_size <= 0:
        raise ValueError(f"block_size must be positive, got {block_size}")
    _no_grad_needed("index_topk", q_idx, centroids)
    dev = N.require_device([q_idx, centroids], "index_topk")
    B, L, d = q_idx.shape
    nb = centroids.shape[1]
    ak = min(top_k, nb)
    idx = torch.zeros(B, L, ak, dtype=torch.long, device=dev)
    scores = None
    if return_scores:
        scores = torch.zeros(B, L, nb, dtype=q_idx.dtype, device=dev)
    if L == 0 or nb == 0:
        return (idx, scores) if return_scores else idx
    rc = N.load().maba_hip_index_topk(N.desc(q_idx), N.desc(centroids), float(lam), int(top_k),
                                      int(block_size), N.desc(idx), N.desc(scores), N.stream_ptr(dev))
    N.check(rc, "index_topk")
    return (idx, scores) if return_scores else idx


@register_kernel("hip", "index_topk_decode")
def hip_index_topk_decode(q, centroids, lambda_dist: float = 0.5, top_k: int = 32,
                          return_scores: bool = False, **kwargs: Any):
    """Decode scoring + top-k over one centroid set per batch (layers/indexer.py:101-112)."""
    lam = kwargs.get("dist_lambda", lambda_dist)
    _no_grad_needed("index_topk_decode", q, centroids)
    dev = N.require_device([q, centroids], "index_topk_decode")
    B, Hq, d = q.shape
    nb = centroids.shape[1]
    ak = min(top_k, nb)
    idx = torch.empty(B, Hq, ak, dtype=torch.long, device=dev)   # every slot is written
    scores = torch.empty(B, Hq, nb, dtype=torch.float32, device=dev) if return_scores else None
    if nb == 0 or B * Hq == 0:
        return (idx, scores) if return_scores else idx
    lib = N.load()
    ws = _workspace(lib.maba_hip_index_topk_decode_workspace_size(B, Hq, nb, int(top_k)), dev)
    rc = lib.maba_hip_index_topk_decode(N.desc(q), N.desc(centroids), float(lam), int(top_k), N.desc(idx),
                                        N.desc(scores), ws.data_ptr(), ws.numel(), N.stream_ptr(dev))
    N.check(rc, "index_topk_decode")
    return (idx, scores) if return_scores else idx


@register_kernel("hip", "stream_superposition")
def hip_stream_superposition(o_local, o_sparse, o_hca, gate_logits=None, gate_weights=None,
                             **kwargs: Any) -> torch.Tensor:
    """Gate superposition (reference contract: dispatcher.py:468-508)."""
    gate = gate_logits if gate_logits is not None else gate_weights
    validate_superposition_inputs(o_local, o_sparse, o_hca, gate)
    if gate is None:
        raise ValueError("Either gate_logits or gate_weights must be provided")
    if gate.dim() not in (3, 4):
        raise ValueError(f"Gate tensor must be 3D or 4D, got {gate.dim()}D")
    _no_grad_needed("stream_superposition", o_local, o_sparse, o_hca, gate)
    dev = N.require_device([o_local, o_sparse, o_hca, gate], "stream_superposition")
    out = torch.empty_like(o_local)
    if o_local.shape[2] == 0 or o_local.numel() == 0:
        return out
    rc = N.load().maba_hip_stream_superposition(N.desc(o_local), N.desc(o_sparse), N.desc(o_hca), N.desc(gate),
                                                int(gate_logits is None), N.desc(out), N.stream_ptr(dev))
    N.check(rc, "stream_superposition")
    return out


@register_kernel("hip", "hca_pool")
def hip_hca_pool(c_kv, pool: int = 64, **kwargs: Any) -> torch.Tensor:
    """Means of complete ``pool``-token latent blocks (layers/sparse_attention.py:206)."""
    _no_grad_needed("hca_pool", c_kv)
    dev = N.require_device([c_kv], "hca_pool")
    B, L, dc = c_kv.shape
    out = torch.empty(B, L // pool, dc, dtype=kwargs.get("out_dtype") or c_kv.dtype, device=dev)
    if out.numel() == 0:
        return out
    rc = N.load().maba_hip_hca_pool(N.desc(c_kv), N.desc(out), int(pool), N.stream_ptr(dev))
    N.check(rc, "hca_pool")
    return out


@register_kernel("hip", "maba_sa_decode")
def hip_maba_sa_decode(q_lat, c_kv, hca, idx, gate, L: int, scale: float, window: int = 128, n_sink: int = 4,
                       block_size: int = 64, pool: int = 64, **kwargs: Any) -> torch.Tensor:
    """Fused local + sparse + HCA decode streams with the gate superposition, in
    latent space (layers/sparse_attention.py:79-219,263-275).  Returns fp32
    ``[B, H, d_c]``; the caller applies the per-head value up-projection."""
    _no_grad_needed("maba_sa_decode", q_lat, c_kv, hca, gate)
    dev = N.require_device([q_lat, c_kv, hca, idx, gate], "maba_sa_decode")
    B, H, dc = q_lat.shape
    out = torch.empty(B, H, dc, dtype=torch.float32, device=dev)
    lib = N.load()
    K = idx.shape[-1]
    ws = _workspace(lib.maba_hip_maba_sa_decode_workspace_size(B, H, dc, int(L), K, int(window), int(n_sink), int(pool)), dev)
    rc = lib.maba_hip_maba_sa_decode(N.desc(q_lat), N.desc(c_kv), N.desc(hca), N.desc(idx), N.desc(gate),
                                     int(L), float(scale), int(window), int(n_sink), int(block_size), int(pool),
                                     N.desc(out), ws.data_ptr(), ws.numel(), N.stream_ptr(dev))
    N.check(rc, "maba_sa_decode")
    return out


@register_kernel("hip", "dgda_prologue")
def hip_dgda_prologue(projections, conv_weights, history=None, n_heads: int = 10, eps: float = 1e-6,
                      gate_dtype: Optional[torch.dtype] = None, with_alpha: bool = True, **kwargs: Any):
    """DGDA layer prologue in one pass (layers/dgda.py:103-121, 186-207): causal depthwise
    conv (kernel 4) + SiLU of q/k/v with the carried history, per-head L2 norm of k, and
    the gate activations.  Same returns as ``common.ref_dgda_prologue``."""
    _no_grad_needed("dgda_prologue", *projections, *conv_weights, *(history or ()))
    dev = N.require_device([*projections, *conv_weights, *(history or ())], "dgda_prologue")
    B, L, C = projections[0].shape
    if C != 64 * n_heads or conv_weights[0].shape[-1] != 4:
        raise NotImplementedError("dgda_prologue: 64-channel heads and kernel 4 only")
    dt = projections[0].dtype
    gdt = gate_dtype or dt
    # three allocations, carved into the outputs (this runs once per layer and decode token)
    qkv = torch.empty(3, B, L, C, dtype=dt, device=dev)
    gates = torch.empty(4 if with_alpha else 3, B, L, C, dtype=gdt, device=dev)
    ys = [qkv[0], qkv[1], qkv[2], gates[0], gates[3] if with_alpha else None, gates[1], gates[2]]
    hdt = history[0].dtype if history is not None else dt
    out_history = kwargs.get("out_history")
    if out_history is not None:   # caller buffers; for one token they may be `history` itself
        nh = list(out_history)
    else:
        nh = list(torch.empty(3, B, C, 3, dtype=hdt, device=dev).unbind(0))
    if L == 0:
        for h, old in zip(nh, history or (None,) * 3):
            h.copy_(old) if old is not None else h.zero_()
        return (*ys, tuple(nh))
    arr = lambda ts: N.desc_array(ts)  # noqa: E731
    rc = N.load().maba_hip_dgda_prologue(arr(projections), arr(conv_weights),
                                         arr(history) if history is not None else None, float(eps), arr(ys),
                                         arr(nh), N.stream_ptr(dev))
    N.check(rc, "dgda_prologue")
    return (*ys, tuple(nh))


@register_kernel("hip", "maba_sa_prefill")
def hip_maba_sa_prefill(q, k, v, kh, vh, early, idx, gate_logits, scale: float, window: int = 128,
                        n_sink: int = 4, block_size: int = 64, pool: int = 64, out_dtype=None,
                        **kwargs: Any) -> torch.Tensor:
    """The three MABA-SA prefill streams and their gate in one launch
    (layers/sparse_attention.py:95-105, 145-171, 173-219, 275): bf16 per-head q, k, v and
    up-projected means, 64-token blocks.  Same contract as ``common.ref_maba_sa_prefill``."""
    _no_grad_needed("maba_sa_prefill", q, k, v, kh, vh, early, gate_logits)
    dev = N.require_device([q, k, v, kh, vh, early, idx, gate_logits], "maba_sa_prefill")
    B, H, Lq, dh = q.shape
    out = torch.empty(B, H, Lq, dh, dtype=out_dtype or q.dtype, device=dev)
    if out.numel() == 0:
        return out
    rc = N.load().maba_hip_maba_sa_prefill(N.desc(q), N.desc(k), N.desc(v), N.desc(kh), N.desc(vh), N.desc(early),
                                           N.desc(idx), N.desc(gate_logits), float(scale), int(window),
                                           int(n_sink), int(block_size), int(pool), N.desc(out),
                                           N.stream_ptr(dev))
    N.check(rc, "maba_sa_prefill")
    return out


# ----------------------------------------------------------------------------- serving path
# Entry points for a decode step whose per-step scalars (the cache position) live in device
# memory, so that one captured HIP graph serves every position.  Not dispatcher ops: the
# reference keeps this code inline (layers/indexer.py:58-112, layers/sparse_attention.py:
# 79-277, model.py:11-128).


def hip_cache_append(c_new, k_new, pos, c_cache, k_cache, hca, centroids, pool: int = 64,
                     block_size: int = 64) -> None:
    """Writes row ``*pos`` of the latent and key caches and the centroid (and, on a completed
    pool-block, the HCA mean) of the block holding it (layers/indexer.py:62-82,
    layers/sparse_attention.py:206).  ``pos`` is a device int64 scalar view."""
    dev = N.require_device([c_new, k_new, pos, c_cache, k_cache, hca, centroids], "cache_append")
    rc = N.load().maba_hip_cache_append(N.desc(c_new), N.desc(k_new), pos.data_ptr(), N.desc(c_cache),
                                        N.desc(k_cache), N.desc(hca), N.desc(centroids), int(pool), int(block_size),
                                        N.stream_ptr(dev))
    N.check(rc, "cache_append")


def hip_cache_append_heads(c_new, k_new, pos, c_cache, k_cache, hca, centroids, q_heads, w_k, gate_in, gate_bias,
                           q_lat, gate_out, pool: int = 64, block_size: int = 64) -> None:
    """``hip_cache_append`` plus, in the same launch, the token's absorbed queries
    ``q_lat [B, H, d_c] = W_k,h^T q_h`` (fp32) for ``q_heads [B, H * d_head]`` and the gate
    logits ``gate_out = gate_in + gate_bias`` (bf16), which the decode streams read next
    (layers/sparse_attention.py:79-219, 274)."""
    dev = N.require_device([c_new, k_new, pos, c_cache, k_cache, hca, centroids, q_heads, w_k, gate_in, gate_bias,
                            q_lat, gate_out], "cache_append_heads")
    rc = N.load().maba_hip_cache_append_heads(N.desc(c_new), N.desc(k_new), pos.data_ptr(), N.desc(c_cache),
                                              N.desc(k_cache), N.desc(hca), N.desc(centroids), int(pool),
                                              int(block_size), N.desc(q_heads), N.desc(w_k), N.desc(gate_in),
                                              N.desc(gate_bias), N.desc(q_lat), N.desc(gate_out), N.stream_ptr(dev))
    N.check(rc, "cache_append_heads")


def hip_index_topk_decode_dev(q, centroids, length, block_size: int, lambda_dist: float, top_k: int,
                              workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Decode scoring + top-k over the first ``ceil(*length / block_size)`` rows of a centroid
    buffer of fixed capacity (layers/indexer.py:101-112); ``length`` is a device int64 scalar
    view and the count must reach ``top_k``."""
    dev = N.require_device([q, centroids, length], "index_topk_decode_dev")
    B, Hq, _ = q.shape
    lib = N.load()
    idx = torch.empty(B, Hq, int(top_k), dtype=torch.long, device=dev)
    nbytes = lib.maba_hip_index_topk_decode_workspace_size(B, Hq, centroids.shape[1], int(top_k))
    ws = workspace if workspace is not None and workspace.numel() >= nbytes else _workspace(nbytes, dev)
    rc = lib.maba_hip_index_topk_decode_dev(N.desc(q), N.desc(centroids), length.data_ptr(), int(block_size),
                                            float(lambda_dist), int(top_k), N.desc(idx), ws.data_ptr(), ws.numel(),
                                            N.stream_ptr(dev))
    N.check(rc, "index_topk_decode_dev")
    return idx


def hip_maba_sa_decode_dev(q_lat, c_cache, hca, idx, gate, length, L_cap: int, scale: float, window: int = 128,
                           n_sink: int = 4, block_size: int = 64, pool: int = 64,
                           workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``maba_sa_decode`` over the first ``*length`` rows of caches of capacity ``L_cap``
    (``length`` a device int64 scalar view); returns fp32 ``[B, H, d_c]``."""
    dev = N.require_device([q_lat, c_cache, hca, idx, gate, length], "maba_sa_decode_dev")
    B, H, dc = q_lat.shape
    lib = N.load()
    out = torch.empty(B, H, dc, dtype=torch.float32, device=dev)
    nbytes = lib.maba_hip_maba_sa_decode_workspace_size(B, H, dc, int(L_cap), idx.shape[-1], int(window),
                                                        int(n_sink), int(pool))
    ws = workspace if workspace is not None and workspace.numel() >= nbytes else _workspace(nbytes, dev)
    rc = lib.maba_hip_maba_sa_decode_dev(N.desc(q_lat), N.desc(c_cache), N.desc(hca), N.desc(idx), N.desc(gate),
                                         length.data_ptr(), int(L_cap), float(scale), int(window), int(n_sink),
                                         int(block_size), int(pool), N.desc(out), ws.data_ptr(), ws.numel(),
                                         N.stream_ptr(dev))
    N.check(rc, "maba_sa_decode_dev")
    return out


def hip_maba_sa_decode_dev_heads(q_lat, c_cache, hca, idx, gate, length, L_cap: int, scale: float, w_v,
                                 out_heads, window: int = 128, n_sink: int = 4, block_size: int = 64, pool: int = 64,
                                 workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``hip_maba_sa_decode_dev`` with each head's value up-projection in its merge launch:
    ``out_heads [B, H * d_head] = W_v,h z_h`` in bf16 (layers/sparse_attention.py:208,
    absorbed).  Returns ``z`` fp32 ``[B, H, d_c]`` as well."""
    dev = N.require_device([q_lat, c_cache, hca, idx, gate, length, w_v, out_heads], "maba_sa_decode_dev_heads")
    B, H, dc = q_lat.shape
    lib = N.load()
    out = torch.empty(B, H, dc, dtype=torch.float32, device=dev)
    nbytes = lib.maba_hip_maba_sa_decode_workspace_size(B, H, dc, int(L_cap), idx.shape[-1], int(window),
                                                        int(n_sink), int(pool))
    ws = workspace if workspace is not None and workspace.numel() >= nbytes else _workspace(nbytes, dev)
    rc = lib.maba_hip_maba_sa_decode_dev_heads(N.desc(q_lat), N.desc(c_cache), N.desc(hca), N.desc(idx),
                                               N.desc(gate), length.data_ptr(), int(L_cap), float(scale),
                                               int(window), int(n_sink), int(block_size), int(pool), N.desc(w_v),
                                               N.desc(out_heads), N.desc(out), ws.data_ptr(), ws.numel(),
                                               N.stream_ptr(dev))
    N.check(rc, "maba_sa_decode_dev_heads")
    return out


def hip_rmsnorm(x, weight, eps: float, mo=None, gate=None, x_out=None) -> torch.Tensor:
    """``RMSNorm(x) * weight`` (model.py:11-22); with ``mo`` and ``gate`` the gated residual
    ``x + gate * mo`` is formed first (written to ``x_out`` when given) and normalised."""
    dev = N.require_device([x, weight, mo, gate, x_out], "rmsnorm")
    h = torch.empty_like(x)
    rc = N.load().maba_hip_rmsnorm(N.desc(x), N.desc(mo), N.desc(gate), N.desc(weight), float(eps), N.desc(x_out),
                                   N.desc(h), N.stream_ptr(dev))
    N.check(rc, "rmsnorm")
    return h


def hip_decode_linear(a, weight, norm_w=None, eps: float = 1e-6, mo=None, gate=None, x_out=None,
                      swiglu: bool = False, rows=None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``A @ weight.T`` for the few rows of one decode token per sequence (``nn.Linear``,
    model.py), with A built in the same launch: ``a``; ``a[rows]`` for a table ``a [V, K]`` and
    int64 ``rows [M]`` / ``[M, 1]`` (an embedding lookup); ``RMSNorm(a) * norm_w``
    (model.py:11-22); ``RMSNorm(a + gate * mo) * norm_w`` with the sum written to ``x_out``
    (the gated residual, model.py:92-128); or, with ``swiglu``, ``silu(a[..., :K]) *
    a[..., K:]`` (model.py:25-38).  bf16 rows ``[M, K]`` or ``[M, 1, K]`` (``[.., 2K]`` for
    swiglu), ``weight [N, K]``; returns bf16 ``[M, N]`` / ``[M, 1, N]`` (``rows``' shape then N;
    into ``out``)."""
    dev = N.require_device([a, rows, weight, norm_w, mo, gate, x_out, out], "decode_linear")
    if out is None:
        lead = rows.shape if rows is not None else a.shape[:-1]
        out = torch.empty(*lead, weight.shape[0], dtype=torch.bfloat16, device=dev)
    rc = N.load().maba_hip_decode_linear(N.desc(a), N.desc(rows), N.desc(mo), N.desc(gate), N.desc(norm_w),
                                         float(eps), 1 if swiglu else 0, N.desc(weight), N.desc(x_out),
                                         N.desc(out), N.stream_ptr(dev))
    N.check(rc, "decode_linear")
    return out


def hip_argmax_rows(x, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``x.argmax(dim=-1, keepdim=True)`` for bf16 / f32 rows ``[M, V]`` or ``[M, 1, V]`` (the
    greedy pick of model.py:279-313): int64 ``[M, 1]`` (into ``out``)."""
    dev = N.require_device([x, out], "argmax_rows")
    if out is None:
        out = torch.empty(x.shape[0], 1, dtype=torch.long, device=dev)
    rc = N.load().maba_hip_argmax_rows(N.desc(x), N.desc(out), N.stream_ptr(dev))
    N.check(rc, "argmax_rows")
    return out


def hip_swiglu(gate_up) -> torch.Tensor:
    """``silu(g) * u`` for ``gate_up = [g | u]`` along the last dim (model.py:25-38)."""
    dev = N.require_device([gate_up], "swiglu")
    out = torch.empty(*gate_up.shape[:-1], gate_up.shape[-1] // 2, dtype=gate_up.dtype, device=dev)
    rc = N.load().maba_hip_swiglu(N.desc(gate_up), N.desc(out), N.stream_ptr(dev))
    N.check(rc, "swiglu")
    return out


def hip_maba_sa_prefill_latent(q_lat, c_kv, hca, idx, gate_logits, scale: float, window: int = 128,
                               n_sink: int = 4, block_size: int = 64, pool: int = 64,
                               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The three MABA-SA prefill streams and their gate in latent form
    (layers/sparse_attention.py:95-105, 145-171, 173-219, 275): query t of ``q_lat [B, Lq, H,
    d_c]`` (``W_k,h^T q_h``, fp32) sits at position ``Lkv - Lq + t`` of the bf16 latent cache
    ``c_kv [B, Lkv, d_c]``; ``hca`` holds its complete-block means.  Returns fp32 ``z [B, Lq, H,
    d_c]`` (into ``out`` when given); the caller applies ``W_v,h``."""
    _no_grad_needed("maba_sa_prefill_latent", q_lat, c_kv, hca, gate_logits)
    dev = N.require_device([q_lat, c_kv, hca, idx, gate_logits], "maba_sa_prefill_latent")
    if out is None:
        out = torch.empty(q_lat.shape, dtype=torch.float32, device=dev)
    if out.numel() == 0:
        return out
    rc = N.load().maba_hip_maba_sa_prefill_latent(N.desc(q_lat), N.desc(c_kv), N.desc(hca), N.desc(idx),
                                                  N.desc(gate_logits), float(scale), int(window), int(n_sink),
                                                  int(block_size), int(pool), N.desc(out), N.stream_ptr(dev))
    N.check(rc, "maba_sa_prefill_latent")
    return out


def hip_dgda_layer_step(projections, conv_weights, history, state, eps: float = 1e-6, out=None):
    """One decode token of the DGDA layer after its input projection (layers/dgda.py:103-121,
    186-207, then the step of dispatcher.py:330-396) in one launch: ``projections`` are the
    six bf16 ``[B, 1, C]`` (or ``[B, C]``) rows, ``history`` the three ``[B, C, 3]`` bf16 conv
    histories and ``state`` the ``[B, H, 64, 64]`` state, both updated in place.  Returns the
    head outputs ``o [B, H, 64]`` in the projections' dtype; equal to ``hip_dgda_prologue``
    followed by ``hip_dgda_step``."""
    dev = N.require_device([*projections, *conv_weights, *history, state], "dgda_layer_step")
    B, C = projections[0].shape[0], projections[0].shape[-1]
    H = C // 64
    if out is None:
        out = torch.empty(B, H, 64, dtype=projections[0].dtype, device=dev)
    hs = N.desc_array(history)
    rc = N.load().maba_hip_dgda_layer_step(N.desc_array(projections), N.desc_array(conv_weights), hs, float(eps),
                                           N.desc(state), N.desc(out), N.desc(state), hs, N.stream_ptr(dev))
    N.check(rc, "dgda_layer_step")
    return out


def hip_dgda_layer_prefill(projections, conv_weights, history=None, eps: float = 1e-6, initial_state=None,
                           out=None, out_history=None, state_dtype: Optional[torch.dtype] = None):
    """The DGDA layer prefill with its prologue fused into the kernels' staging
    (layers/dgda.py:103-121, 186-233): from the six bf16 projections ``[B, L, C]`` straight to
    the head outputs and the final state, q/k/v and the gates never stored.  Returns ``(o
    [B, L, C] bf16, final state [B, H, 64, 64], new conv history (3 x [B, C, 3]))``; ``out``
    may be a preallocated ``[B, L, C]`` buffer, ``out_history`` the new history's buffers."""
    _no_grad_needed("dgda_layer_prefill", *projections, *conv_weights, *(history or ()), initial_state)
    dev = N.require_device([*projections, *conv_weights, *(history or ()), initial_state], "dgda_layer_prefill")
    B, L, C = projections[0].shape
    H = C // 64
    if out is None:
        out = torch.empty(B, L, C, dtype=projections[0].dtype, device=dev)
    state = torch.empty(B, H, 64, 64, dtype=state_dtype or projections[0].dtype, device=dev)
    nh = list(out_history) if out_history is not None else \
        list(torch.empty(3, B, C, 3, dtype=projections[0].dtype, device=dev).unbind(0))
    lib = N.load()
    ws = _workspace(lib.maba_hip_dgda_layer_prefill_workspace_size(B, H, L), dev)
    o4 = out.view(B, L, H, 64).transpose(1, 2)   # the kernel's [B, H, L, 64] view of the [B, L, C] rows
    rc = lib.maba_hip_dgda_layer_prefill(N.desc_array(projections), N.desc_array(conv_weights),
                                         N.desc_array(history) if history is not None else None, float(eps),
                                         N.desc(initial_state), N.desc(o4), N.desc(state), N.desc_array(nh),
                                         ws.data_ptr(), ws.numel(), N.stream_ptr(dev))
    N.check(rc, "dgda_layer_prefill")
    return out, state, tuple(nh)
