"""DGDA (decoupled gated delta attention) oracle -- TEST INFRASTRUCTURE ONLY.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg.  Never imported by the product package.

Math (per batch ``b`` and head ``h``; ``S`` is ``[dk, dv]``, gates are per
channel: ``alpha_t, b_t`` in R^dk, ``w_t`` in R^dv)::

    S'    = diag(alpha_t) S                      (common.py:258)
    pred  = (b_t * k_t)^T S'                     (common.py:259-260)
    delta = w_t * v_t - pred                     (common.py:261-262)
    S_t   = S' + k_t delta^T                     (common.py:263)
    o_t   = S_t^T q_t                            (common.py:264)

Functions
---------
``dgda_prefill_seq``     token loop of ``ref_dgda_prefill`` (common.py:229-268),
                         float64.  Pinned by: closed-form single-token case,
                         alpha=0 wipes the state (test_cpu_dgda.py:143-157),
                         b=w=0 freezes it (test_cpu_dgda.py:210-230), L=1
                         prefill == step (test_cpu_dgda.py:472-495),
                         chunk chaining (test_triton_dgda.py:162-180), a
                         dense-matrix brute-force restatement on tiny shapes
                         and the golden vectors in ``tests/golden``.
``dgda_step``            one token, ``ref_dgda_step`` (common.py:271-309).
                         Pinned by equality with ``dgda_prefill_seq`` at L=1
                         and the hand-computed golden vector.
``dgda_prefill_chunked`` chunked WY/UT algorithm of ``cpu_dgda_prefill``
                         (cpu_dgda.py:82-197) with exact triangular solves.
                         Pinned against ``dgda_prefill_seq`` (chunk-size
                         independence, test_dgda.py:122-137) and the
                         all-ones analytic inverse (test_dgda_precision.py:
                         102-129).
``layer_prologue``       the DGDA layer's op inputs from its projections
                         (layers/dgda.py:103-121 conv + SiLU with carried
                         history, :193-197 gates, :207 key norm), float64
                         loops.  Pinned by: identity and pure-shift conv
                         kernels (the conv reduces to SiLU of the input, or of
                         the input three tokens back through the history),
                         softplus/sigmoid closed forms at 0 and the -14 clamp,
                         unit-norm keys, and prefill-then-continue equal to one
                         pass (the history carry).
"""
from __future__ import annotations

import numpy as np


def _decay(alpha, log_alpha):
    """Decay factors as the sequential reference takes them.

    ``ref_dgda_prefill`` uses ``alpha`` when it is given and ``exp(log_alpha)``
    otherwise (common.py:242-243).
    """
    if alpha is not None:
        return np.asarray(alpha, dtype=np.float64)
    if log_alpha is None:
        raise ValueError("Either alpha or log_alpha must be provided")
    return np.exp(np.asarray(log_alpha, dtype=np.float64))


def dgda_prefill_seq(q, k, v, alpha=None, b=None, w=None, initial_state=None,
                     log_alpha=None):
    """Token-sequential DGDA prefill in float64 (common.py:229-268).

    Shapes: q, k, alpha, b ``[B,H,L,dk]``; v, w ``[B,H,L,dv]``;
    initial_state ``[B,H,dk,dv]`` or None (zeros).  Returns ``(o, S)`` with
    ``o [B,H,L,dv]`` and ``S [B,H,dk,dv]``, both float64.
    """
    if b is None or w is None:
        raise ValueError("Both b and w gate tensors must be provided")
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    b = np.asarray(b, np.float64)
    w = np.asarray(w, np.float64)
    a = _decay(alpha, log_alpha)
    B, H, L, dk = q.shape
    dv = v.shape[-1]
    if initial_state is None:
        S = np.zeros((B, H, dk, dv), np.float64)
    else:
        S = np.array(initial_state, dtype=np.float64, copy=True)
    out = np.empty((B, H, L, dv), np.float64)
    for t in range(L):
        Sd = a[:, :, t, :, None] * S                                  # common.py:258
        pred = np.einsum("bhk,bhkv->bhv", b[:, :, t] * k[:, :, t], Sd)  # common.py:259-260
        delta = w[:, :, t] * v[:, :, t] - pred                        # common.py:261-262
        S = Sd + k[:, :, t, :, None] * delta[:, :, None, :]           # common.py:263
        out[:, :, t] = np.einsum("bhk,bhkv->bhv", q[:, :, t], S)      # common.py:264
    return out, S


def dgda_step(q, k, v, alpha=None, b=None, w=None, state=None, log_alpha=None):
    """One decode step (common.py:271-309); accepts ``[B,H,d]`` or ``[B,H,1,d]``."""
    def sq(x):
        if x is None:
            return None
        x = np.asarray(x, np.float64)
        return x[:, :, 0] if x.ndim == 4 and x.shape[2] == 1 else x
    q, k, v, b, w = sq(q), sq(k), sq(v), sq(b), sq(w)
    a = _decay(sq(alpha), sq(log_alpha))
    B, H, dk = q.shape
    dv = v.shape[-1]
    S = np.zeros((B, H, dk, dv)) if state is None else np.asarray(state, np.float64)
    Sd = a[..., None] * S                                            # common.py:302
    pred = np.einsum("bhk,bhkv->bhv", b * k, Sd)                     # common.py:303-304
    delta = w * v - pred                                             # common.py:305-306
    S_new = Sd + k[..., None] * delta[..., None, :]                  # common.py:307
    out = np.einsum("bhk,bhkv->bhv", q, S_new)                       # common.py:308
    return out, S_new


def _chunk_log_alpha(alpha, log_alpha):
    """Log-decay as the chunked CPU backend takes it (cpu_dgda.py:63-68).

    ``log_alpha`` wins when given and is clamped to ``[-46, 0]``; otherwise
    ``log(clamp(alpha, 1e-20, 1))``.
    """
    if log_alpha is not None:
        return np.clip(np.asarray(log_alpha, np.float64), -46.0, 0.0)
    return np.log(np.clip(np.asarray(alpha, np.float64), 1e-20, 1.0))


def dgda_prefill_chunked(q, k, v, alpha=None, b=None, w=None, chunk_size=16,
                         initial_state=None, log_alpha=None, dtype=np.float64):
    """Chunked WY/UT DGDA prefill (cpu_dgda.py:82-197), exact triangular solve.

    Per chunk with inclusive cumulative log-decay ``Lam`` (cpu_dgda.py:101-107):
    ``D_ij = exp(min(Lam_i - Lam_j, 0))``, ``L = tril_strict(sum_d bk_i D_ij k_j)``,
    ``A = tril(sum_d q_i D_ij k_j)``, ``v_e = w*v - (bk*e^Lam) S0``,
    ``u = (I+L)^-1 v_e``, ``o = (q*e^Lam) S0 + A u``,
    ``S = e^{Lam_C} S0 + (k*e^{Lam_C-Lam})^T u`` (cpu_dgda.py:116-146).
    The remainder chunk uses the same formulas (cpu_dgda.py:148-194).
    """
    f = lambda x: np.asarray(x, dtype)
    q, k, v, b, w = f(q), f(k), f(v), f(b), f(w)
    la = _chunk_log_alpha(alpha, log_alpha).astype(dtype)
    B, H, L, dk = q.shape
    dv = v.shape[-1]
    S = np.zeros((B, H, dk, dv), dtype) if initial_state is None else f(initial_state).copy()
    outs = np.empty((B, H, L, dv), dtype)
    for s in range(0, L, chunk_size):
        e = min(L, s + chunk_size)
        n = e - s
        qc, kc, vc, bc, wc, lc = (x[:, :, s:e] for x in (q, k, v, b, w, la))
        cla = np.cumsum(lc, axis=2)                                   # [B,H,n,dk]
        diff = cla[:, :, :, None, :] - cla[:, :, None, :, :]          # [B,H,n,n,dk]
        dec = np.exp(np.minimum(diff, 0.0))
        bk = bc * kc
        lmat = np.tril(np.einsum("bhid,bhijd,bhjd->bhij", bk, dec, kc), -1)
        amat = np.tril(np.einsum("bhid,bhijd,bhjd->bhij", qc, dec, kc), 0)
        lam = np.exp(cla)
        ve = wc * vc - np.einsum("bhid,bhdv->bhiv", bk * lam, S)
        eye = np.eye(n, dtype=dtype)
        u = np.linalg.solve(eye + lmat, ve)                           # exact solve
        outs[:, :, s:e] = np.einsum("bhid,bhdv->bhiv", qc * lam, S) + amat @ u
        dte = np.exp(cla[:, :, -1:, :] - cla)
        S = np.exp(cla[:, :, -1, :])[..., None] * S + np.einsum("bhid,bhiv->bhdv", kc * dte, u)
    return outs, S


def dgda_prefill_dense(q, k, v, alpha=None, b=None, w=None, initial_state=None,
                       log_alpha=None):
    """Brute-force restatement for tiny shapes, used only to pin the token loop.

    Writes the recurrence with explicit matrices per token,
    ``S_t = (I - k_t (b_t*k_t)^T) diag(alpha_t) S_{t-1} + k_t (w_t*v_t)^T``,
    unrolled from its transition/affine form rather than the einsum form of
    ``dgda_prefill_seq``.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    b = np.asarray(b, np.float64)
    w = np.asarray(w, np.float64)
    a = _decay(alpha, log_alpha)
    B, H, L, dk = q.shape
    dv = v.shape[-1]
    o = np.zeros((B, H, L, dv))
    Sf = np.zeros((B, H, dk, dv))
    for bi in range(B):
        for hi in range(H):
            S = np.zeros((dk, dv)) if initial_state is None else np.array(initial_state[bi, hi], np.float64)
            for t in range(L):
                kt = k[bi, hi, t].reshape(dk, 1)
                ct = (b[bi, hi, t] * k[bi, hi, t]).reshape(dk, 1)
                trans = (np.eye(dk) - kt @ ct.T) @ np.diag(a[bi, hi, t])
                S = trans @ S + kt @ (w[bi, hi, t] * v[bi, hi, t]).reshape(1, dv)
                o[bi, hi, t] = (q[bi, hi, t].reshape(1, dk) @ S).ravel()
            Sf[bi, hi] = S
    return o, Sf


def layer_prologue(xq, xk, xv, xa, xb, xw, wq, wk, wv, hist=None, n_heads=10, eps=1e-6):
    """DGDA layer prologue in float64 (reference layers/dgda.py:103-121, 186-207).

    x* : [B, L, C] projections; w* : [C, K] depthwise conv taps (cross-correlation, as
    torch's conv1d: y_t = sum_j w[j] p[t + j] over p = [history, x]); hist: None or
    three [B, C, K-1] carried inputs, oldest first.  Returns q, k, v, log_alpha, alpha,
    b, w ([B, L, C]) and the three new histories [B, C, K-1]."""
    def silu(z):
        return z / (1.0 + np.exp(-z))

    outs, hists = [], []
    for i, (x, w) in enumerate(((xq, wq), (xk, wk), (xv, wv))):
        x = np.asarray(x, np.float64)
        w = np.asarray(w, np.float64)
        B, L, C = x.shape
        K = w.shape[1]
        h = np.zeros((B, C, K - 1)) if hist is None else np.asarray(hist[i], np.float64)
        p = np.concatenate([h, x.transpose(0, 2, 1)], axis=2)          # [B, C, K-1+L]
        y = np.zeros((B, L, C))
        for t in range(L):
            for j in range(K):
                y[:, t, :] += w[None, :, j] * p[:, :, t + j]
        outs.append(silu(y))
        hists.append(p[:, :, p.shape[2] - (K - 1):].copy())
    q, k, v = outs
    B, L, C = q.shape
    kh = k.reshape(B, L, n_heads, C // n_heads)
    k = (kh / (np.sqrt((kh * kh).sum(-1, keepdims=True)) + eps)).reshape(B, L, C)
    xa = np.asarray(xa, np.float64)
    softplus = np.where(xa > 20.0, xa, np.log1p(np.exp(np.minimum(xa, 20.0))))
    la = np.maximum(-softplus, -14.0)
    sig = lambda z: 1.0 / (1.0 + np.exp(-np.asarray(z, np.float64)))  # noqa: E731
    return q, k, v, la, np.exp(la), sig(xb), sig(xw), hists
