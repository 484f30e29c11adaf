"""MABA-SA layer: the caller of the indexer, the three attention streams and the
gate superposition (reference: layers/sparse_attention.py:11-277).

Decode (one token): everything runs in latent space through the fused
``maba_sa_decode`` op.  ``q_lat[b,h] = W_k,h^T q[b,h]`` (absorbed key
up-projection), the op returns ``z[b,h] = sum_s g_s sum_j p_sj c_j`` over the
latent rows of the local window + sinks, the indexer's gathered blocks and the
HCA block means, and the layer applies ``W_v,h`` and ``o_proj``.  This replaces
the reference's per-step concatenation of per-head K/V caches
(sparse_attention.py:241-261) and its per-step re-pooling of the whole latent
cache (:206): HCA means are kept and extended by one mean per completed block.
``LatentCache`` additionally offers a preallocated latent cache for serving loops
(``decode_step``), avoiding the O(L) ``torch.cat`` that the reference's
``forward(x, past_c_kv)`` interface implies.

Prefill (several tokens) follows the reference streams: causal sliding window + sinks
(:95-105), per-query gathered blocks (:145-171), HCA over complete-block means with the
early running-mean rule (:173-219), then ``stream_superposition``.  In bf16 without
gradients one fused launch does all three streams and the gate, in latent form or in head
space (``_prefill_form`` picks); otherwise the dense torch path runs.
"""
from __future__ import annotations

import math
from typing import Any, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from maba_sparse.kernels.dispatcher import (dispatch_hca_pool, dispatch_maba_sa_decode, dispatch_maba_sa_prefill,
                                            dispatch_stream_superposition, get_backend)
from maba_sparse.layers._wcache import WeightCacheMixin, cached
from maba_sparse.layers.indexer import DGIndexer, _Growing

# Fused prefill: the head-space kernel is taken while 16 consecutive queries list fewer than
# this many distinct blocks, in units of top_k (the measured crossover with the latent kernel)
PREFILL_UNION_LIMIT = 5.25


class LatentCache:
    """Preallocated decode state of one layer: latent rows ``[B, capacity, d_c]`` and
    the means of their complete ``pool``-token blocks."""

    def __init__(self, batch: int, capacity: int, d_c: int, pool: int = 64,
                 device=None, dtype: torch.dtype = torch.float32) -> None:
        self.c = torch.empty(batch, capacity, d_c, device=device, dtype=dtype)
        self.hca = torch.empty(batch, max(1, capacity // pool), d_c, device=device, dtype=dtype)
        self.pool = pool
        self.n = 0       # latent rows held
        self.nh = 0      # complete-block means held

    def append(self, c_new: torch.Tensor) -> None:
        m = c_new.shape[1]
        if self.n + m > self.c.shape[1]:
            raise ValueError(f"LatentCache full: {self.n} + {m} > {self.c.shape[1]}")
        self.c[:, self.n: self.n + m] = c_new.to(self.c.dtype)
        self.n += m
        full = self.n // self.pool
        if full > self.nh:
            lo, hi = self.nh * self.pool, full * self.pool
            self.hca[:, self.nh: full] = dispatch_hca_pool(self.c[:, lo:hi], pool=self.pool)
            self.nh = full


class DeviceCache:
    """Decode caches of one MABA-SA layer for the serving path, in the format the
    ``cache_append`` kernel maintains (all bf16, capacity ``cap`` tokens):
    latent rows ``c [B, cap, d_c]``, indexer keys ``keys [B, cap, d_idx]``, the means of the
    complete 64-token blocks ``hca [B, cap // 64, d_c]`` and the block centroids
    ``cent [B, ceil(cap / 64), d_idx]`` (the last one the zero-padded tail centroid while its
    block is incomplete).  The sequence length lives in a device counter shared by the
    model's layers, so one captured decode step replays at every position."""

    def __init__(self, c_kv: torch.Tensor, keys: torch.Tensor, cap: int, pool: int = 64, block: int = 64) -> None:
        from maba_sparse.kernels import hip_backend as hb
        B, L, dc = c_kv.shape
        di = keys.shape[2]
        dev, dt = c_kv.device, c_kv.dtype
        self.cap, self.pool, self.block = cap, pool, block
        self.c = torch.zeros(B, cap, dc, device=dev, dtype=dt)
        self.keys = torch.zeros(B, cap, di, device=dev, dtype=dt)
        self.hca = torch.zeros(B, max(1, cap // pool), dc, device=dev, dtype=dt)
        self.cent = torch.zeros(B, (cap + block - 1) // block, di, device=dev, dtype=dt)
        self.c[:, :L] = c_kv
        self.keys[:, :L] = keys.to(dt)
        if L >= pool:
            self.hca[:, : L // pool] = hb.hip_hca_pool(c_kv[:, : (L // pool) * pool], pool=pool)
        if L > 0:
            self.cent[:, : (L + block - 1) // block] = hb.hip_compute_centroids(self.keys[:, :L], block_size=block)


class MabaSparseAttention(WeightCacheMixin, nn.Module):
    def __init__(self, config: Optional[Any] = None, dim: int = 640, n_heads: int = 10, d_head: int = 64,
                 d_c: int = 128, window_size: int = 128, block_size: int = 64, top_k: int = 32,
                 hca_pool_size: int = 64, dist_lambda: float = 0.5, d_idx: int = 64,
                 ablation_mode: str = "full") -> None:
        super().__init__()
        g = (lambda n, alt, d: getattr(config, n, getattr(config, alt, d)) if alt else getattr(config, n, d)) \
            if config is not None else (lambda n, alt, d: d)
        self.dim = g("dim", "d_model", dim)
        self.n_heads = g("n_heads", "num_heads", n_heads)
        self.d_head = g("d_head", None, d_head)
        self.d_c = g("d_c", None, d_c)
        self.window_size = g("window_size", None, window_size)
        self.block_size = g("block_size", None, block_size)
        self.top_k = g("top_k", None, top_k)
        self.hca_pool_size = g("hca_pool_size", None, hca_pool_size)
        self.dist_lambda = g("dist_lambda", None, dist_lambda)
        self.n_sink_tokens = g("n_sink_tokens", None, 4)
        d_idx = g("d_idx", None, d_idx)
        self.ablation_mode = ablation_mode if ablation_mode is not None else g("ablation_mode", None, "full")
        self.scale = 1.0 / math.sqrt(self.d_head)
        H, dh = self.n_heads, self.d_head
        self.q_proj = nn.Linear(self.dim, H * dh, bias=False)
        self.kv_down_proj = nn.Linear(self.dim, self.d_c, bias=False)
        self.k_up_proj = nn.Linear(self.d_c, H * dh, bias=False)
        self.v_up_proj = nn.Linear(self.d_c, H * dh, bias=False)
        self.o_proj = nn.Linear(H * dh, self.dim, bias=False)
        self.stream_gate = nn.Linear(self.dim, 3, bias=True)
        self.indexer = DGIndexer(dim=self.dim, d_idx=d_idx, block_size=self.block_size, top_k=self.top_k,
                                 dist_lambda=self.dist_lambda)
        self._hca_means: Optional[_Growing] = None
        # fused bf16 prefill: "auto" picks the latent or the head-space kernel from the
        # selections' sharing (see _prefill_form); the union limit is in units of top_k
        self.prefill_form = "auto"
        self.prefill_union_limit = PREFILL_UNION_LIMIT
        self._install_weight_cache_hooks()

    def reset_cache(self) -> None:
        self.indexer.reset_cache()
        self._hca_means = None

    def get_gate_weights(self, x: torch.Tensor) -> torch.Tensor:
        return F.softmax(self.stream_gate(x), dim=-1)

    # ------------------------------------------------------------ decode (fused)
    def _f32_heads(self, lin: nn.Linear, key: str) -> torch.Tensor:
        """``lin.weight`` in fp32 as ``[H, d_head, d_c]``, converted again only after the weight
        changes (decode calls this twice per token)."""
        w = lin.weight
        return cached(self, key, (w,), lambda: w.float().view(self.n_heads, self.d_head, self.d_c))

    def _absorbed_query(self, x: torch.Tensor) -> torch.Tensor:
        """``W_k,h^T q_h`` for the single token of ``x [B, 1, dim]`` -> ``[B, H, d_c]`` fp32."""
        B = x.shape[0]
        q = self.q_proj(x).view(B, self.n_heads, self.d_head).float()
        return torch.einsum("bhd,hdc->bhc", q, self._f32_heads(self.k_up_proj, "_wk_f32"))

    def _heads_out(self, z: torch.Tensor, dtype: torch.dtype, decode_linear: bool = False) -> torch.Tensor:
        """``W_v,h z_h`` then ``o_proj``; ``z [B, H, d_c]`` -> ``[B, 1, dim]`` (``o_proj`` as a
        HIP decode linear with ``decode_linear``)."""
        B = z.shape[0]
        Wv = self._f32_heads(self.v_up_proj, "_wv_f32")
        o = torch.einsum("bhc,hdc->bhd", z.float(), Wv).reshape(B, 1, self.n_heads * self.d_head).to(dtype)
        if decode_linear:
            from maba_sparse.kernels import hip_backend as hb
            return hb.hip_decode_linear(o, self.o_proj.weight)
        return self.o_proj(o)

    def _hca_for(self, c_full: torch.Tensor) -> torch.Tensor:
        """Complete-block means of ``c_full``, extended incrementally across decode steps."""
        L, r = c_full.shape[1], self.hca_pool_size
        full = L // r
        h = self._hca_means
        if h is not None and h.shape[0] == c_full.shape[0] and full - 1 <= h.n <= full:
            if h.n == full - 1:
                h.append(dispatch_hca_pool(c_full[:, (full - 1) * r: full * r], pool=r))
        else:
            self._hca_means = _Growing(dispatch_hca_pool(c_full, pool=r)) if full > 0 else None
        if self._hca_means is None:
            return c_full.new_zeros(c_full.shape[0], 1, self.d_c)
        return self._hca_means.view()

    def _decode(self, x: torch.Tensor, c_all: torch.Tensor, L: int, hca: torch.Tensor,
                idx: torch.Tensor, q: Optional[torch.Tensor] = None,
                gate_logits: Optional[torch.Tensor] = None) -> torch.Tensor:
        q_lat = self._absorbed_query(x) if q is None else torch.einsum(
            "bhd,hdc->bhc", q.reshape(x.shape[0], self.n_heads, self.d_head).float(),
            self._f32_heads(self.k_up_proj, "_wk_f32"))
        gl = self.stream_gate(x) if gate_logits is None else gate_logits
        z = dispatch_maba_sa_decode(q_lat, c_all, hca, idx, gl.view(-1, 3),
                                    L=L, scale=self.scale, window=self.window_size, n_sink=self.n_sink_tokens,
                                    block_size=self.block_size, pool=self.hca_pool_size)
        return self._heads_out(z, x.dtype)

    def _token_projections(self, x: torch.Tensor, proj=None, gate_bias: bool = True):
        """q, the new latent, the indexer's query and key and the gate logits of one token from
        one GEMM over the stacked weights (the stack is rebuilt only after a weight changes).

        The indexer query comes first and the stack is padded with zero rows to a multiple of
        eight, so that the query view starts at the GEMM output's base with a row stride that is
        a multiple of eight elements: the bf16 MFMA decode scoring requires 16-byte aligned query
        rows and takes a scalar kernel otherwise."""
        mods = (self.indexer.q_idx_proj, self.indexer.k_idx_proj, self.q_proj, self.kv_down_proj, self.stream_gate)
        ws = [m.weight for m in mods]
        sizes = [w.shape[0] for w in ws]
        pad = -sum(sizes) % 8

        def stack():
            st = torch.cat(ws, dim=0)
            return torch.cat([st, st.new_zeros(pad, st.shape[1])], dim=0) if pad else st

        w5 = cached(self, "w5", ws, stack)
        y = proj(w5) if proj is not None else F.linear(x, w5)
        qi, ki, q, c_new, gl, _ = y.split(sizes + [pad], dim=-1)
        return q, c_new, qi, ki, (gl + self.stream_gate.bias if gate_bias else gl)

    def decode_step(self, x: torch.Tensor, cache: LatentCache,
                    past_centroids: Optional[torch.Tensor] = None) -> torch.Tensor:
        """One decode token over a preallocated ``LatentCache`` (appends this token's latent)."""
        if x.shape[1] != 1:
            raise ValueError("decode_step takes one token")
        if torch.is_grad_enabled() and any(p.requires_grad for p in self.parameters()):
            cache.append(self.kv_down_proj(x))
            idx, _ = self.indexer(x, return_scores=False, past_centroids=past_centroids)
            hca = cache.hca[:, : max(cache.nh, 1)]
            return self._decode(x, cache.c, cache.n, hca, idx)
        q, c_new, qi, ki, gl = self._token_projections(x)
        cache.append(c_new)
        idx, _ = self.indexer.forward_projected(qi, ki, return_scores=False, past_centroids=past_centroids)
        hca = cache.hca[:, : max(cache.nh, 1)]
        return self._decode(x, cache.c, cache.n, hca, idx, q=q, gate_logits=gl)

    def decode_step_device(self, x: torch.Tensor, cache: DeviceCache, counters: torch.Tensor,
                           return_parts: bool = False, proj=None):
        """One token on the serving path: the token's row joins ``cache`` at position
        ``counters[0]`` (device), the decode indexer and the fused three-stream decode run over
        the first ``counters[1] = counters[0] + 1`` rows.  Same math as ``decode_step``; HIP
        backend, bf16 caches and at least ``top_k`` blocks of history.  ``return_parts`` also
        returns the selected blocks and the latent-space output ``z`` (for tests).
        ``proj(weight)``, when given, stands for ``F.linear(x, weight)`` of the layer input
        (a decode linear that builds its normalised input in the same launch; ``x`` then only
        gives the batch and dtype), and ``o_proj`` runs as a decode linear too."""
        from maba_sparse.kernels import hip_backend as hb
        B = x.shape[0]
        if x.dtype == torch.bfloat16 and self._heads_fusable():
            # five launches for the streams: the append also forms the absorbed queries and the
            # gate logits, the merge also applies each head's value up-projection
            q, c_new, qi, ki, gl = self._token_projections(x, proj, gate_bias=False)
            q_lat = torch.empty(B, self.n_heads, self.d_c, dtype=torch.float32, device=x.device)
            gate = torch.empty(B, 3, dtype=torch.bfloat16, device=x.device)
            hb.hip_cache_append_heads(c_new[:, 0], ki[:, 0], counters[0], cache.c, cache.keys, cache.hca, cache.cent,
                                      q[:, 0], self.k_up_proj.weight, gl[:, 0], self.stream_gate.bias, q_lat, gate,
                                      pool=self.hca_pool_size, block_size=self.block_size)
            idx = hb.hip_index_topk_decode_dev(qi, cache.cent, counters[1], self.block_size, self.dist_lambda,
                                               self.top_k)
            o = torch.empty(B, 1, self.n_heads * self.d_head, dtype=torch.bfloat16, device=x.device)
            z = hb.hip_maba_sa_decode_dev_heads(q_lat, cache.c, cache.hca, idx, gate, counters[1], cache.cap,
                                                self.scale, self.v_up_proj.weight, o[:, 0],
                                                window=self.window_size, n_sink=self.n_sink_tokens,
                                                block_size=self.block_size, pool=self.hca_pool_size)
            out = hb.hip_decode_linear(o, self.o_proj.weight) if proj is not None else self.o_proj(o)
            return (out, idx, z) if return_parts else out
        q, c_new, qi, ki, gl = self._token_projections(x, proj)
        hb.hip_cache_append(c_new[:, 0], ki[:, 0], counters[0], cache.c, cache.keys, cache.hca, cache.cent,
                            pool=self.hca_pool_size, block_size=self.block_size)
        idx = hb.hip_index_topk_decode_dev(qi, cache.cent, counters[1], self.block_size, self.dist_lambda, self.top_k)
        q_lat = torch.einsum("bhd,hdc->bhc", q.reshape(B, self.n_heads, self.d_head).float(),
                             self._f32_heads(self.k_up_proj, "_wk_f32"))
        z = hb.hip_maba_sa_decode_dev(q_lat, cache.c, cache.hca, idx, gl.view(-1, 3), counters[1], cache.cap,
                                      self.scale, window=self.window_size, n_sink=self.n_sink_tokens,
                                      block_size=self.block_size, pool=self.hca_pool_size)
        out = self._heads_out(z, x.dtype, decode_linear=proj is not None)
        return (out, idx, z) if return_parts else out

    def _heads_fusable(self) -> bool:
        """Whether the serving step's append and merge launches also form the absorbed queries,
        the gate logits and the value up-projection: bf16 weights, a gate bias, heads of at most
        64 channels."""
        ws = (self.k_up_proj.weight, self.v_up_proj.weight, self.stream_gate.weight)
        return (all(w.dtype == torch.bfloat16 for w in ws) and self.stream_gate.bias is not None
                and self.stream_gate.bias.dtype == torch.bfloat16 and self.d_head <= 64
                and self.k_up_proj.bias is None and self.v_up_proj.bias is None)

    # ------------------------------------------------------------ prefill (HIP)
    def _prefill_fusable(self, q: torch.Tensor, c_full: torch.Tensor, idx: torch.Tensor) -> bool:
        """Whether the one-launch HIP prefill takes this call: the ``hip`` backend, bf16, the
        kernel's head sizes and 64-token blocks, no gradients and the full three streams."""
        if q.device.type != "cuda" or get_backend(q.device) != "hip" or self.ablation_mode == "no_hca":
            return False
        if q.dtype != torch.bfloat16 or c_full.dtype != torch.bfloat16:
            return False
        if self.block_size != 64 or idx.shape[-1] > 64 or c_full.shape[1] > (1 << 20):
            return False
        if self.d_c % 32 != 0 or self.d_c > 128 or self.n_heads > 16:
            return False
        return not (torch.is_grad_enabled() and any(p.requires_grad for p in self.parameters()))

    def _prefill_form(self, idx: torch.Tensor) -> str:
        """``"latent"`` or ``"heads"`` for a fused prefill with selections ``idx [B, Lq, K]``.

        The latent kernel does each query's tiles on its own (the ten heads share every key row,
        as at decode); the head-space kernel gives each run of 64 queries the union of their
        blocks, staged once per tile and computed by each 16-query wave that lists it (16
        queries share every key tile, per head).  Its cost grows with the union of 16
        consecutive queries' blocks, the latent kernel's does not: measured at 10 heads of 64,
        d_c 128, top-32, the two are equal near 5.25 K distinct blocks per 16 queries (random
        queries at 32k tokens give 5.1 K, at 64k 6.5 K, at 128k 7.6 K), and neighbouring queries
        of a trained or randomly initialised model select nearly the same blocks (about 3 K, where
        the head-space kernel is 2.5 times faster).  The union is counted on the GPU from ``idx``
        (one segmented sort); ``self.prefill_form`` may force either."""
        if self.prefill_form != "auto":
            return self.prefill_form
        B, Lq, K = idx.shape
        if Lq == 1:   # one selection shared by every query
            return "heads"
        if Lq < 16:
            return "latent"
        grp = idx[:, : (Lq // 16) * 16].reshape(B, Lq // 16, 16 * K).sort(dim=-1).values
        distinct = (grp[..., 1:] != grp[..., :-1]).sum(dim=-1).float().mean().item() + 1.0
        return "heads" if distinct < self.prefill_union_limit * K else "latent"

    def _fused_prefill(self, x, q, c_full, idx):
        if self._prefill_form(idx) == "heads" and self.d_head in (32, 64, 128):
            return self._fused_prefill_heads(x, q, c_full, idx)
        return self._fused_prefill_latent(x, q, c_full, idx)

    def _fused_prefill_latent(self, x, q, c_full, idx):
        """The three streams and the gate in latent form: ``q_lat = W_k,h^T q_h`` per query, one
        ``maba_sa_prefill_latent`` launch over the bf16 latent rows and their complete-block
        means, then ``o_h = W_v,h z_h``.  Keys and values are never up-projected (the cache is
        read once per query tile instead of materialising ``[B, H, Lkv, dh]`` twice).
        Returns ``[B, H, Lq, dh]`` (a transposed view)."""
        from maba_sparse.kernels import hip_backend as hb
        b, h, lq, dh = q.shape
        r = self.hca_pool_size
        nc = c_full.shape[1] // r
        Wk = self._f32_heads(self.k_up_proj, "_wk_f32")
        Wv = self._f32_heads(self.v_up_proj, "_wv_f32")
        q_lat = torch.einsum("bhtd,hdc->bthc", q.float(), Wk)
        hca = (hb.hip_hca_pool(c_full[:, : nc * r], pool=r) if nc > 0
               else c_full.new_zeros(b, 1, self.d_c))
        z = hb.hip_maba_sa_prefill_latent(q_lat.contiguous(), c_full.contiguous(), hca, idx, self.stream_gate(x),
                                          scale=self.scale, window=self.window_size, n_sink=self.n_sink_tokens,
                                          block_size=self.block_size, pool=r)
        return torch.einsum("bthc,hdc->bthd", z, Wv).transpose(1, 2)

    def _fused_prefill_heads(self, x, q, c_full, idx):
        """The streams' inputs as the dense path forms them (per-head keys and values, the
        up-projected complete-block means, the running-mean rows before ``pool - 1``), then
        one ``maba_sa_prefill`` launch with the gate.  Returns ``[B, H, Lq, dh]``."""
        b, h, lq, dh = q.shape
        lkv = c_full.shape[1]
        heads = lambda t, n: t.view(b, n, h, dh).transpose(1, 2)  # noqa: E731
        k = heads(self.k_up_proj(c_full), lkv)
        v = heads(self.v_up_proj(c_full), lkv)
        r = self.hca_pool_size
        nc = lkv // r
        kh = vh = None
        if nc > 0:
            means = c_full[:, : nc * r].reshape(b, nc, r, self.d_c).mean(dim=2)
            kh, vh = heads(self.k_up_proj(means), nc), heads(self.v_up_proj(means), nc)
        off = lkv - lq
        n_early = max(0, min(lq, r - 1 - off))
        early = None
        if n_early > 0:
            cm = torch.cumsum(c_full[:, : off + n_early], dim=1)
            cm = cm / torch.arange(1, cm.shape[1] + 1, device=x.device).view(1, -1, 1)
            early = heads(self.v_up_proj(cm[:, off: off + n_early]), n_early)
        return dispatch_maba_sa_prefill(q, k, v, kh, vh, early, idx, self.stream_gate(x), scale=self.scale,
                                        window=self.window_size, n_sink=self.n_sink_tokens,
                                        block_size=self.block_size, pool=r)

    # ------------------------------------------------------------ prefill (dense)
    def _dense_streams(self, x, q, c_full, idx):
        b, h, lq, dh = q.shape
        lkv = c_full.shape[1]
        k = self.k_up_proj(c_full).view(b, lkv, h, dh).transpose(1, 2)
        v = self.v_up_proj(c_full).view(b, lkv, h, dh).transpose(1, 2)
        pos = (lkv - lq) + torch.arange(lq, device=x.device)          # absolute query positions
        j = torch.arange(lkv, device=x.device)

        def masked_attend(scores, mask, vals):
            p = torch.nan_to_num(F.softmax(scores.masked_fill(~mask, float("-inf")), dim=-1), nan=0.0)
            return p @ vals

        # local: causal, within the window or one of the sinks
        keep = (j[None] <= pos[:, None]) & (((pos[:, None] - j[None]) < self.window_size) |
                                             (j[None] < min(self.n_sink_tokens, lkv)))
        ol = masked_attend((q @ k.transpose(-1, -2)) * self.scale, keep[None, None], v)

        # sparse: per query, the tokens of its selected blocks that are < L and <= its position
        bs = self.block_size
        nb = (lkv + bs - 1) // bs
        ak = idx.shape[-1]
        pad = nb * bs - lkv
        kb = F.pad(k, (0, 0, 0, pad)).view(b, h, nb, bs, dh)
        vb = F.pad(v, (0, 0, 0, pad)).view(b, h, nb, bs, dh)
        os_ = torch.zeros_like(ol)
        for t0 in range(0, lq, 128):
            t1 = min(t0 + 128, lq)
            bi = idx[:, t0:t1] if idx.shape[1] == lq else idx[:, :1].expand(b, t1 - t0, ak)
            sel = bi.reshape(b, 1, -1, 1, 1).expand(b, h, (t1 - t0) * ak, bs, dh)
            ks = torch.gather(kb, 2, sel).view(b, h, t1 - t0, ak * bs, dh)
            vs = torch.gather(vb, 2, sel).view(b, h, t1 - t0, ak * bs, dh)
            tok = (bi[..., None] * bs + torch.arange(bs, device=x.device)).reshape(b, t1 - t0, ak * bs)
            ok = (tok < lkv) & (tok <= pos[t0:t1, None])
            s = (q[:, :, t0:t1, None, :] @ ks.transpose(-1, -2)).squeeze(-2) * self.scale
            p = torch.nan_to_num(F.softmax(s.masked_fill(~ok[:, None], float("-inf")), dim=-1), nan=0.0)
            os_[:, :, t0:t1] = (p[..., None, :] @ vs).squeeze(-2)

        # HCA: complete-block means whose last token is <= the query; running mean before that
        r = self.hca_pool_size
        oh = torch.zeros_like(ol)
        if self.ablation_mode != "no_hca":
            early = pos < (r - 1)
            if early.any():
                cm = torch.cumsum(c_full[:, : int(pos[early].max()) + 1], dim=1)
                cm = cm / torch.arange(1, cm.shape[1] + 1, device=x.device).view(1, -1, 1)
                oh[:, :, early] = self.v_up_proj(cm[:, pos[early]]).view(b, -1, h, dh).transpose(1, 2)
            nc = lkv // r
            if (~early).any() and nc > 0:
                means = c_full[:, : nc * r].reshape(b, nc, r, self.d_c).mean(dim=2)
                kh = self.k_up_proj(means).view(b, nc, h, dh).transpose(1, 2)
                vh = self.v_up_proj(means).view(b, nc, h, dh).transpose(1, 2)
                ends = (torch.arange(nc, device=x.device) + 1) * r - 1
                late = ~early
                ok = ends[None] <= pos[late][:, None]
                oh[:, :, late] = masked_attend((q[:, :, late] @ kh.transpose(-1, -2)) * self.scale,
                                               ok[None, None], vh)
        return ol, os_, oh

    def forward(self, x: torch.Tensor, past_c_kv: Optional[torch.Tensor] = None,
                past_centroids: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        b, l, _ = x.shape
        ic = self.indexer._cached_k_idx
        if past_c_kv is None or (ic is not None and ic.shape[1] != past_c_kv.shape[1]):
            self.reset_cache()
        c_kv = self.kv_down_proj(x)
        c_full = torch.cat([past_c_kv, c_kv], dim=1) if past_c_kv is not None else c_kv
        idx, _ = self.indexer(x, return_scores=False, past_centroids=past_centroids)
        if l == 1 and self.ablation_mode != "no_hca":
            return self._decode(x, c_full, c_full.shape[1], self._hca_for(c_full), idx), c_full
        q = self.q_proj(x).view(b, l, self.n_heads, self.d_head).transpose(1, 2)
        if self._prefill_fusable(q, c_full, idx):
            o = self._fused_prefill(x, q, c_full, idx)
        else:
            ol, os_, oh = self._dense_streams(x, q, c_full, idx)
            o = dispatch_stream_superposition(ol, os_, oh, gate_logits=self.stream_gate(x))
        if l > 1 and not self.training and self.ablation_mode != "no_hca":
            self._hca_for(c_full)       # seed the incremental means for the decode steps
        o = o.transpose(1, 2).reshape(b, l, self.n_heads * self.d_head).to(q.dtype)
        return self.o_proj(o), c_full


MABASALayer = MabaSparseAttention
