"""DGDA layer: the caller of ``dgda_prefill`` / ``dgda_step`` (reference: layers/dgda.py:22-287).

The layer produces the op inputs exactly as the reference does and calls the
dispatcher with the same keywords, so the ``"hip"`` backend receives the
reference's call pattern:

* q, k, v projections, each followed by a causal depthwise conv (kernel 4) and
  SiLU with a carried history of the last ``kernel_size - 1`` inputs
  (dgda.py:103-121);
* gates ``b = sigmoid``, ``w = sigmoid``, ``log_alpha = max(-softplus, -14)``,
  ``alpha = exp(log_alpha)``, both decay forms passed (dgda.py:193-197, 221-233);
* k L2-normalised with ``+eps`` on the norm (dgda.py:207);
* q/k/v and gates as ``[B, T, H, d]`` storage viewed ``[B, H, T, d]``
  (dgda.py:199-205), which the HIP kernels read in place.

Constructor arguments, parameter names and the ``ConvState`` layout match the
reference so that its state dicts and conv states can be used unchanged.
"""
from __future__ import annotations

from typing import Any, Optional, Sequence, Tuple, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

from maba_sparse.layers._wcache import WeightCacheMixin, cached
from maba_sparse.kernels.dispatcher import (dispatch_dgda_prefill, dispatch_dgda_prologue, dispatch_dgda_step,
                                            get_backend)


class ConvState(tuple):
    """(q_hist, k_hist, v_hist), each ``[B, channels, kernel_size - 1]`` (layers/dgda.py:10-19)."""

    @property
    def shape(self) -> torch.Size:
        if not self:
            return torch.Size([0, 0, 0, 0])
        first = self[0]
        return torch.Size([first.shape[0], len(self), first.shape[1], first.shape[2]])

    def as_tensor(self) -> torch.Tensor:
        return torch.stack(tuple(self), dim=1)


def _cfg(config: Any, names: Sequence[str], default: Any) -> Any:
    for n in names:
        if config is not None and hasattr(config, n):
            return getattr(config, n)
    return default


class DGDALayer(WeightCacheMixin, nn.Module):
    def __init__(self, config: Optional[Any] = None, dim: int = 640, n_heads: int = 10,
                 d_head: Optional[int] = None, kernel_size: int = 4, eps: float = 1e-6) -> None:
        super().__init__()
        self.dim = _cfg(config, ("dim", "d_model"), dim)
        self.n_heads = _cfg(config, ("n_heads", "num_heads"), n_heads)
        self.d_head = _cfg(config, ("d_head",), d_head) or self.dim // self.n_heads
        self.d_k = _cfg(config, ("d_k",), self.d_head)
        self.d_v = _cfg(config, ("d_v",), self.d_head)
        self.kernel_size = _cfg(config, ("kernel_size", "conv_kernel_size"), kernel_size)
        self.k_size = self.kernel_size
        self.eps = _cfg(config, ("eps", "rms_norm_eps"), eps)
        self.chunk_size = _cfg(config, ("chunk_size",), 16)
        self.inversion_method = _cfg(config, ("inversion_method",), "adaptive")
        self.adaptive_tol = _cfg(config, ("adaptive_tol",), 7e-5)
        # bf16 prefill on the HIP backend: the prologue runs inside the recurrence kernels
        # (False: the one-pass prologue kernel, then the op on its stored outputs)
        self.fuse_prologue = True

        qk, vd = self.n_heads * self.d_k, self.n_heads * self.d_v
        lin = lambda i, o: nn.Linear(i, o, bias=False)  # noqa: E731
        dw = lambda c: nn.Conv1d(c, c, self.kernel_size, groups=c, bias=False, padding=0)  # noqa: E731
        self.q_proj, self.k_proj, self.v_proj = lin(self.dim, qk), lin(self.dim, qk), lin(self.dim, vd)
        self.conv_q, self.conv_k, self.conv_v = dw(qk), dw(qk), dw(vd)
        self.gate_alpha, self.gate_erase, self.gate_write = lin(self.dim, qk), lin(self.dim, qk), lin(self.dim, vd)
        self.o_proj = lin(vd, self.dim)
        for m in (self.q_proj, self.k_proj, self.v_proj, self.gate_alpha, self.gate_erase, self.gate_write,
                  self.o_proj):
            nn.init.xavier_uniform_(m.weight)
        for m in (self.conv_q, self.conv_k, self.conv_v):
            nn.init.normal_(m.weight, mean=0.0, std=0.02)
        self._install_weight_cache_hooks()

    # reference aliases (layers/dgda.py:78-88)
    alpha_proj = property(lambda self: self.gate_alpha)
    b_proj = property(lambda self: self.gate_erase)
    w_proj = property(lambda self: self.gate_write)

    # ------------------------------------------------------------------ conv
    def _conv_silu(self, x: torch.Tensor, conv: nn.Conv1d,
                   hist: Optional[torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor]:
        """Causal depthwise conv + SiLU of ``x [B, L, C]``; returns (y, new history)."""
        kh = self.kernel_size - 1
        xt = x.transpose(1, 2)
        if hist is None:
            seq = F.pad(xt, (kh, 0)) if kh > 0 else xt
        else:
            if hist.shape[-1] < kh:
                hist = F.pad(hist, (kh - hist.shape[-1], 0))
            elif hist.shape[-1] > kh:
                hist = hist[..., hist.shape[-1] - kh:]
            seq = torch.cat([hist, xt], dim=2)
        new_hist = seq[..., seq.shape[-1] - kh:].contiguous() if kh > 0 else seq[..., :0].contiguous()
        return F.silu(conv(seq)).transpose(1, 2), new_hist

    def _split_conv_state(self, cs, B: int, device, dtype):
        """Accepts the conv-state forms the reference accepts (layers/dgda.py:123-164)."""
        if cs is None:
            return None, None, None
        to = lambda t: None if t is None else t.to(device=device, dtype=dtype)  # noqa: E731
        kh = max(self.kernel_size - 1, 0)
        if isinstance(cs, (tuple, list)):
            if len(cs) == 3:
                return to(cs[0]), to(cs[1]), to(cs[2])
            if len(cs) == 1 and isinstance(cs[0], (tuple, list)):
                return to(cs[0][0]), to(cs[0][1]), to(cs[0][2])
        if isinstance(cs, torch.Tensor):
            if cs.dim() == 4 and cs.shape[1] == 3:
                return to(cs[:, 0]), to(cs[:, 1]), to(cs[:, 2])
            if cs.dim() == 5 and cs.shape[1] == 3:
                t = cs.reshape(B, 3, cs.shape[2], kh)
                return to(t[:, 0]), to(t[:, 1]), to(t[:, 2])
            flat = cs.reshape(B, -1, kh)
            qk, vd = self.n_heads * self.d_k, self.n_heads * self.d_v
            n = flat.shape[1]
            if n == 2 * qk + vd:
                return to(flat[:, :qk]), to(flat[:, qk:2 * qk]), to(flat[:, 2 * qk:])
            if n == qk and qk != vd:
                return to(flat), to(flat), torch.zeros(B, vd, kh, device=device, dtype=dtype)
            return to(flat), to(flat), to(flat)
        raise ValueError(f"Unsupported conv_state shape or type: {type(cs)}")

    # ---------------------------------------------------------------- inputs
    def _prologue_fusable(self, x: torch.Tensor) -> bool:
        """Whether the one-pass HIP prologue takes this call: the ``hip`` backend, the
        model's head shape (64-channel heads, kernel 4), f32/bf16 and no gradients."""
        if x.device.type != "cuda" or get_backend(x.device) != "hip":
            return False
        if self.kernel_size != 4 or self.d_k != 64 or self.d_v != 64 or self.n_heads > 16:
            return False
        if x.dtype not in (torch.float32, torch.bfloat16):
            return False
        return not (torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())))

    def _projections(self, x: torch.Tensor, hists):
        """One GEMM for the six projections (``[B, L, C]`` views, row stride 6C) and the carried
        conv history cut or zero-padded to ``kernel_size - 1`` taps (None without one)."""
        C = self.n_heads * self.d_k
        ws = [m.weight for m in (self.q_proj, self.k_proj, self.v_proj, self.gate_alpha, self.gate_erase,
                                 self.gate_write)]
        # restacked only after a weight changes (one stack per input dtype)
        w6 = cached(self, f"w6_{x.dtype}", ws, lambda: torch.cat(ws, dim=0).to(x.dtype))
        projs = F.linear(x, w6).split(C, dim=-1)
        kh = self.kernel_size - 1
        hist = None
        if hists[0] is not None:
            fit = lambda h: F.pad(h, (kh - h.shape[-1], 0)) if h.shape[-1] < kh else h[..., h.shape[-1] - kh:]  # noqa: E731
            hist = tuple(fit(h) for h in hists)
        return projs, hist

    def _fused_forward(self, x: torch.Tensor, state, hists):
        """The bf16 prefill with the prologue fused into the recurrence kernels' staging: the
        six projections go straight to the head outputs, q/k/v and the gates are never
        stored (one GEMM, the HIP passes, ``o_proj``)."""
        from maba_sparse.kernels import hip_backend as hb
        projs, hist = self._projections(x, hists)
        convs = (self.conv_q.weight, self.conv_k.weight, self.conv_v.weight)
        s0 = state.to(x.dtype) if state is not None else None
        o, S, nh = hb.hip_dgda_layer_prefill(projs, convs, hist, eps=self.eps, initial_state=s0)
        return self.o_proj(o), S, ConvState(nh)

    def _fused_op_inputs(self, x: torch.Tensor, state, hists):
        """One GEMM for the six projections, then the HIP prologue (conv + SiLU, gates, key
        norm) in one pass.  Gates come out in fp32 (the chunked kernels' gate format, more
        precise than the reference's cast to the module dtype), so the op is called with
        ``allow_mixed_dtypes``."""
        B, L, _ = x.shape
        H, dk = self.n_heads, self.d_k
        projs, hist = self._projections(x, hists)
        q, k, v, la, _, b, w, nh = dispatch_dgda_prologue(
            projs, (self.conv_q.weight, self.conv_k.weight, self.conv_v.weight), hist, n_heads=H, eps=self.eps,
            gate_dtype=torch.float32, with_alpha=False)
        heads = lambda t: t.view(B, L, H, dk).transpose(1, 2)  # noqa: E731
        # the op takes log_alpha when both decay forms are given (common.py:242-243 computes
        # alpha = exp(log_alpha) when only log_alpha is given), so alpha is not materialised
        args = dict(q=heads(q), k=heads(k), v=heads(v), alpha=None, b=heads(b), w=heads(w),
                    log_alpha=heads(la), allow_mixed_dtypes=True)
        if state is not None:
            state = state.to(x.dtype)
        return args, state, ConvState(nh)

    def _op_inputs(self, x: torch.Tensor, state, conv_state):
        """Projections, convs, gates and head-major views -- the op's keyword arguments."""
        B, L, _ = x.shape
        H, dk, dv = self.n_heads, self.d_k, self.d_v
        hq, hk, hv = self._split_conv_state(conv_state, B, x.device, x.dtype)
        if self._prologue_fusable(x):
            return self._fused_op_inputs(x, state, (hq, hk, hv))
        q, nq = self._conv_silu(self.q_proj(x), self.conv_q, hq)
        k, nk = self._conv_silu(self.k_proj(x), self.conv_k, hk)
        v, nv = self._conv_silu(self.v_proj(x), self.conv_v, hv)
        log_alpha = torch.clamp(-F.softplus(self.gate_alpha(x)), min=-14.0)
        heads = lambda t, d: t.view(B, L, H, d).transpose(1, 2)  # noqa: E731  [B,T,H,d] viewed [B,H,T,d]
        q = heads(q, dk)
        k = heads(k, dk)
        k = k / (torch.linalg.vector_norm(k, dim=-1, keepdim=True) + self.eps)
        dt = q.dtype
        args = dict(q=q, k=k.to(dt), v=heads(v, dv).to(dt),
                    alpha=heads(torch.exp(log_alpha), dk).to(dt),
                    b=heads(torch.sigmoid(self.gate_erase(x)), dk).to(dt),
                    w=heads(torch.sigmoid(self.gate_write(x)), dv).to(dt),
                    log_alpha=heads(log_alpha, dk).to(dt))
        if state is not None:
            state = state.to(dt)
        return args, state, ConvState((nq, nk, nv))

    # ---------------------------------------------------------------- public
    def forward(self, x: torch.Tensor, state: Optional[torch.Tensor] = None,
                conv_state: Optional[Union[torch.Tensor, Tuple[torch.Tensor, ...]]] = None,
                chunk_size: Optional[int] = None,
                inversion_method: Optional[str] = None) -> Tuple[torch.Tensor, torch.Tensor, ConvState]:
        B, L, D = x.shape
        H, dk, dv = self.n_heads, self.d_k, self.d_v
        if L == 0:   # layers/dgda.py:178-184
            kh = max(self.kernel_size - 1, 0)
            zq = torch.zeros(B, H * dk, kh, dtype=x.dtype, device=x.device)
            zv = torch.zeros(B, H * dv, kh, dtype=x.dtype, device=x.device)
            st = state.clone() if state is not None else torch.zeros(B, H, dk, dv, dtype=x.dtype, device=x.device)
            return torch.empty(B, 0, D, dtype=x.dtype, device=x.device), st, ConvState((zq, zq, zv))
        if self._prologue_fusable(x) and x.dtype == torch.bfloat16 and self.fuse_prologue:
            hists = self._split_conv_state(conv_state, B, x.device, x.dtype)
            if hists[0] is None or all(h.dtype == torch.bfloat16 for h in hists):
                return self._fused_forward(x, state, hists)
        args, state, ncs = self._op_inputs(x, state, conv_state)
        o, S = dispatch_dgda_prefill(
            **args,
            chunk_size=chunk_size if chunk_size is not None else self.chunk_size,
            initial_state=state,
            inversion_method=inversion_method if inversion_method is not None else self.inversion_method,
            adaptive_tol=self.adaptive_tol,
        )
        o = o.transpose(1, 2).reshape(B, L, H * dv)
        return self.o_proj(o), S, ncs

    def step(self, x: torch.Tensor, state: Optional[torch.Tensor] = None,
             conv_state: Optional[Union[torch.Tensor, Tuple[torch.Tensor, ...]]] = None
             ) -> Tuple[torch.Tensor, torch.Tensor, ConvState]:
        B, L = x.shape[0], x.shape[1]
        if L != 1:
            raise ValueError(f"step() takes one token, got {L}")
        args, state, ncs = self._op_inputs(x, state, conv_state)
        oh, S = dispatch_dgda_step(**args, state=state)
        return self.o_proj(oh.reshape(B, 1, self.n_heads * self.d_v)), S, ncs


    def step_device(self, x: torch.Tensor, state: torch.Tensor, hists, proj=None) -> torch.Tensor:
        """One token on the serving path: the prologue writes the new conv history over
        ``hists`` (three ``[B, C, 3]`` buffers) and the step updates ``state`` in place, so a
        captured launch sequence replays with the same buffers at every position.  Same math
        as ``step``; HIP backend only.  ``proj(weight)``, when given, stands for ``F.linear(x,
        weight)`` of the layer input (a decode linear that builds its normalised input in the
        same launch; ``x`` then only gives the batch and dtype), and ``o_proj`` runs as a
        decode linear too."""
        from maba_sparse.kernels import hip_backend as hb
        B = x.shape[0]
        H, dk, dv = self.n_heads, self.d_k, self.d_v
        ws = [m.weight for m in (self.q_proj, self.k_proj, self.v_proj, self.gate_alpha, self.gate_erase,
                                 self.gate_write)]
        w6 = cached(self, f"w6_{x.dtype}", ws, lambda: torch.cat(ws, dim=0).to(x.dtype))
        projs = (proj(w6) if proj is not None else F.linear(x, w6)).split(H * dk, dim=-1)
        convs = (self.conv_q.weight, self.conv_k.weight, self.conv_v.weight)
        if (self.fuse_prologue and dk == dv == 64 and convs[0].shape[-1] == 4 and x.dtype == torch.bfloat16
                and all(h.dtype == torch.bfloat16 for h in hists)):
            # prologue and step in one launch; state and history updated in place
            o = hb.hip_dgda_layer_step(projs, convs, tuple(hists), state, eps=self.eps).reshape(B, 1, H * dv)
            return hb.hip_decode_linear(o, self.o_proj.weight) if proj is not None else self.o_proj(o)
        q, k, v, la, _, b, w, _ = hb.hip_dgda_prologue(
            projs, (self.conv_q.weight, self.conv_k.weight, self.conv_v.weight), tuple(hists), n_heads=H,
            eps=self.eps, gate_dtype=torch.float32, with_alpha=False, out_history=tuple(hists))
        o, _ = hb.hip_dgda_step(q.view(B, H, dk), k.view(B, H, dk), v.view(B, H, dv), log_alpha=la.view(B, H, dk),
                                b=b.view(B, H, dk), w=w.view(B, H, dv), state=state, new_state=state,
                                allow_mixed_dtypes=True)
        o = o.reshape(B, 1, H * dv)
        return hb.hip_decode_linear(o.to(x.dtype), self.o_proj.weight) if proj is not None else self.o_proj(o)


DecoupledGatedDeltaAttention = DGDALayer
