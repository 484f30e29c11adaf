"""DGDA on host cores: the ``cpu`` backend's prefill and decode step.

The prefill is the chunked WY form of the reference's CPU kernels
(reference kernels/cpu_dgda.py:33-197): per chunk of ``chunk_size`` tokens with the
inclusive cumulative log-decay ``Lam`` (a vector over key channels),

    L = tril_strict(sum_d (b k)_i e^{min(Lam_i - Lam_j, 0)} k_j),  A = tril(sum_d q_i ... k_j)
    v_e = w v - (b k e^Lam) S,   u = (I + L)^-1 v_e,   o = (q e^Lam) S + A u,
    S' = e^{Lam_last} S + (k e^{Lam_last - Lam})^T u,

with the reference's inversion methods ("exact": the triangular solve; "adaptive": the
third-order Neumann series I - L + L^2 - L^3, then the exact solve for a chunk whose residual
exceeds ``adaptive_tol``; any other name: the series alone, as cpu_dgda.py:113-134 treats it).  The state-independent parts are
formed for a block of chunks at a time, so the ``[.., C, C, dk]`` decay tensor never
exceeds about 64 MB (the reference forms it for the whole sequence at once); the
recurrence then walks the chunks of the block.  A ragged tail is padded with zero tokens of
zero log-decay, which leave the state unchanged.  Arithmetic in fp32 (fp64 inputs stay
fp64), results in the input dtype; torch's intra-op threads use the host cores.
"""
from __future__ import annotations

from typing import Any, Optional, Tuple

import torch

from maba_sparse.kernels.common import validate_dgda_prefill_inputs, validate_dgda_step_inputs

_BLOCK_BYTES = 64 << 20   # bound on the per-block decay tensor


def _work_dtype(t: torch.Tensor) -> torch.dtype:
    return torch.float32 if t.dtype in (torch.float16, torch.bfloat16) else t.dtype


def _log_decay(alpha, log_alpha):
    """The reference's decay forms (cpu_dgda.py:63-68), branch for branch: log_alpha alone is
    taken as given; alpha alone as log(alpha clamped to [1e-20, 1]); both given, log_alpha
    clamped to [-46, 0].  (Within a chunk every decay ratio is clamped to <= 1 below, as in the
    reference, so a growing gate only counts across chunk boundaries.)"""
    if log_alpha is None:
        return torch.log(alpha.clamp(min=1e-20, max=1.0))
    if alpha is None:
        return log_alpha
    return torch.clamp(log_alpha, min=-46.0, max=0.0)


def cpu_dgda_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, alpha: Optional[torch.Tensor] = None,
                     b: Optional[torch.Tensor] = None, w: Optional[torch.Tensor] = None, chunk_size: int = 16,
                     initial_state: Optional[torch.Tensor] = None, log_alpha: Optional[torch.Tensor] = None,
                     inversion_method: str = "adaptive", adaptive_tol: float = 7e-5,
                     **kwargs: Any) -> Tuple[torch.Tensor, torch.Tensor]:
    """Chunked DGDA prefill on the CPU (reference kernels/cpu_dgda.py:33-197; contract of
    ``dgda_prefill``, dispatcher.py:258-327).  Returns ``(o [B,H,L,dv], S [B,H,dk,dv])``."""
    validate_dgda_prefill_inputs(q, k, v, alpha, b, w, initial_state, log_alpha=log_alpha)
    orig = q.dtype
    wd = _work_dtype(q)
    B, H, L, dk = q.shape
    dv = v.shape[-1]
    S = (torch.zeros(B, H, dk, dv, dtype=wd, device=q.device) if initial_state is None
         else initial_state.to(wd).clone())
    if L == 0:
        return torch.empty(B, H, 0, dv, dtype=orig, device=q.device), S.to(orig)
    la = _log_decay(None if alpha is None else alpha.to(wd), None if log_alpha is None else log_alpha.to(wd))
    q, k, v = q.to(wd), k.to(wd), v.to(wd)
    b = b.to(wd).expand(B, H, L, dk)
    w = w.to(wd).expand(B, H, L, dv)
    la = la.expand(B, H, L, dk)
    C = int(chunk_size)
    nch = -(-L // C)
    pad = nch * C - L
    if pad:
        padded = lambda t: torch.nn.functional.pad(t, (0, 0, 0, pad))  # noqa: E731  zero tokens at the end
        q, k, v, b, w, la = (padded(t) for t in (q, k, v, b, w, la))
    out = torch.empty(B, H, nch * C, dv, dtype=wd, device=q.device)
    per_chunk = B * H * C * C * dk * torch.finfo(wd).bits // 8
    G = max(1, min(nch, _BLOCK_BYTES // max(per_chunk, 1)))
    eye = torch.eye(C, dtype=wd, device=q.device)
    for c0 in range(0, nch, G):
        g = min(G, nch - c0)
        sl = slice(c0 * C, (c0 + g) * C)
        blk = lambda t: t[:, :, sl].reshape(B, H, g, C, t.shape[-1])  # noqa: E731
        qc, kc, vc, bc, wc, lc = (blk(t) for t in (q, k, v, b, w, la))
        cla = torch.cumsum(lc, dim=-2)                                        # [B,H,g,C,dk]
        dec = torch.exp(torch.clamp(cla.unsqueeze(-2) - cla.unsqueeze(-3), max=0.0))   # [B,H,g,C,C,dk]
        bk = bc * kc
        l_mat = torch.tril(torch.einsum("bhgid,bhgijd,bhgjd->bhgij", bk, dec, kc), diagonal=-1)
        a_mat = torch.tril(torch.einsum("bhgid,bhgijd,bhgjd->bhgij", qc, dec, kc), diagonal=0)
        del dec
        lam = torch.exp(cla)
        bh = bk * lam
        ql = qc * lam
        wv = wc * vc
        last = cla[..., -1:, :]
        kd = kc * torch.exp(last - cla)
        ds0 = torch.exp(last).transpose(-1, -2)                              # [B,H,g,dk,1]
        if inversion_method == "exact":
            inv = torch.linalg.solve_triangular(eye + l_mat, eye.expand_as(l_mat), upper=False)
        else:
            l2 = l_mat @ l_mat
            inv = eye - l_mat + l2 - l2 @ l_mat
        for j in range(g):
            ve = wv[:, :, j] - bh[:, :, j] @ S
            u = inv[:, :, j] @ ve
            if inversion_method == "adaptive":
                r = ve - u - l_mat[:, :, j] @ u
                if r.abs().max() > adaptive_tol or not torch.isfinite(u).all():
                    u = torch.linalg.solve_triangular(eye + l_mat[:, :, j], ve, upper=False)
            t0 = (c0 + j) * C
            out[:, :, t0:t0 + C] = ql[:, :, j] @ S + a_mat[:, :, j] @ u
            S = ds0[:, :, j] * S + kd[:, :, j].transpose(-1, -2) @ u
    return out[:, :, :L].to(orig), S.to(orig)


def cpu_dgda_step(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, alpha: Optional[torch.Tensor] = None,
                  b: Optional[torch.Tensor] = None, w: Optional[torch.Tensor] = None,
                  state: Optional[torch.Tensor] = None, log_alpha: Optional[torch.Tensor] = None,
                  **kwargs: Any) -> Tuple[torch.Tensor, torch.Tensor]:
    """One DGDA token on the CPU (reference kernels/cpu_dgda.py:200-261): S' = alpha S +
    k (w v - (b k) (alpha S)), o = q S', in fp32 for half-precision inputs."""
    validate_dgda_step_inputs(q, k, v, alpha, b, w, state, log_alpha=log_alpha)
    orig = q.dtype
    wd = _work_dtype(q)
    if alpha is None:
        alpha = torch.exp(log_alpha.to(wd))
    q, k, v, alpha, b, w = (t.to(wd) for t in (q, k, v, alpha, b, w))
    if q.dim() == 4 and q.shape[2] == 1:
        q, k, v, alpha, b, w = (t.squeeze(2) for t in (q, k, v, alpha, b, w))
    B, H, dk = q.shape
    dv = v.shape[-1]
    S = torch.zeros(B, H, dk, dv, dtype=wd, device=q.device) if state is None else state.to(wd)
    sd = alpha.unsqueeze(-1) * S
    pred = ((b * k).unsqueeze(-2) @ sd).squeeze(-2)
    new_state = sd + k.unsqueeze(-1) * (w * v - pred).unsqueeze(-2)
    o = (q.unsqueeze(-2) @ new_state).squeeze(-2)
    return o.to(orig), new_state.to(orig)
