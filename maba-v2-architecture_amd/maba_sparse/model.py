"""The Maba v2 causal LM around the hot-path layers: the full-model decode harness.

Mirrors ``maba_sparse/model.py`` of the reference (``:11-313``): RMSNorm, SwiGLU FFN,
factorised embeddings tied to the LM head, blocks in a 3:1 pattern (every fourth block
is MABA-SA, the others DGDA) with sigmoid-gated residuals, ``forward`` (prefill, returning
per-layer states) and ``step`` (one token).  ``generate_greedy`` is the serving loop: one
prefill, then single-token steps in which the DGDA blocks carry their recurrent and conv
states and the MABA-SA blocks decode over a preallocated ``LatentCache`` (incremental
latent rows, HCA means and indexer centroids) instead of the reference's per-step
``torch.cat`` of the whole cache (``model.py:280-313`` with ``sparse_attention.py:241-261``).
The multi-token-prediction head and the loss are training-side and are not built here.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, List, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from maba_sparse.layers._wcache import WeightCacheMixin, cached
from maba_sparse.kernels.dispatcher import get_backend
from maba_sparse.layers.dgda import DGDALayer
from maba_sparse.layers.sparse_attention import DeviceCache, LatentCache, MabaSparseAttention


@dataclass
class MabaConfig:
    """The fields of the reference's ``MabaSparseConfig`` (config.py:5-38) the stack reads."""
    dim: int = 640
    n_layers: int = 20
    n_heads: int = 10
    d_head: int = 64
    vocab_size: int = 32768
    d_emb: int = 128
    kernel_size: int = 4
    chunk_size: int = 16
    eps: float = 1e-6
    d_c: int = 128
    d_idx: int = 64
    block_size: int = 64
    window_size: int = 128
    top_k: int = 32
    hca_pool_size: int = 64
    dist_lambda: float = 0.5
    intermediate_size: int = 1248
    rms_norm_eps: float = 1e-6
    residual_gate_bias: float = 2.0


def get_101m_config(**overrides: Any) -> MabaConfig:
    """The 101M configuration (reference model.py:165-181): 20 layers, d_model 640, 10 heads,
    factorised 32768 -> 128 -> 640 embedding, SwiGLU width 1248."""
    return MabaConfig(**overrides)


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.dim = dim
        self.eps = max(float(eps), 1e-6)
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.rms_norm(x, (self.dim,), self.weight, eps=self.eps)


def _frozen(module: nn.Module, key: str, fn, *params: torch.Tensor) -> torch.Tensor:
    """``fn(*params)``, kept on ``module`` until a parameter changes (see ``layers/_wcache.py``).
    For inference: under autograd the value is recomputed."""
    return cached(module, key, params, lambda: fn(*params))


class SwiGLUFFN(WeightCacheMixin, nn.Module):
    def __init__(self, dim: int, intermediate_size: int) -> None:
        super().__init__()
        self.w_gate = nn.Linear(dim, intermediate_size, bias=False)
        self.w_up = nn.Linear(dim, intermediate_size, bias=False)
        self.w_down = nn.Linear(intermediate_size, dim, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # gate and up projections as one GEMM over the stacked weights
        w = _frozen(self, "gate_up", lambda a, b: torch.cat([a, b], dim=0), self.w_gate.weight, self.w_up.weight)
        g, u = F.linear(x, w).chunk(2, dim=-1)
        return self.w_down(F.silu(g) * u)

    def forward_hip(self, x: torch.Tensor) -> torch.Tensor:
        """``forward`` with the activation ``silu(g) * u`` as one HIP kernel."""
        from maba_sparse.kernels import hip_backend as hb
        w = _frozen(self, "gate_up", lambda a, b: torch.cat([a, b], dim=0), self.w_gate.weight, self.w_up.weight)
        return self.w_down(hb.hip_swiglu(F.linear(x, w)))


class FactorizedEmbeddings(nn.Module):
    def __init__(self, vocab_size: int, d_emb: int, dim: int) -> None:
        super().__init__()
        self.in_emb = nn.Embedding(vocab_size, d_emb)
        self.proj = nn.Linear(d_emb, dim, bias=False)

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        return self.proj(self.in_emb(input_ids))


class MabaBlock(WeightCacheMixin, nn.Module):
    def __init__(self, config: MabaConfig, layer_idx: int) -> None:
        super().__init__()
        self.layer_idx = layer_idx
        self.is_attention = (layer_idx + 1) % 4 == 0
        self.norm1 = RMSNorm(config.dim, eps=config.rms_norm_eps)
        self.mixer = MabaSparseAttention(config) if self.is_attention else DGDALayer(config)
        self.norm2 = RMSNorm(config.dim, eps=config.rms_norm_eps)
        self.ffn = SwiGLUFFN(config.dim, config.intermediate_size)
        self.res_gate1 = nn.Parameter(torch.full((config.dim,), config.residual_gate_bias))
        self.res_gate2 = nn.Parameter(torch.full((config.dim,), config.residual_gate_bias))

    def _residual(self, x: torch.Tensor, mo: torch.Tensor) -> torch.Tensor:
        g1 = _frozen(self, "g1", torch.sigmoid, self.res_gate1)
        g2 = _frozen(self, "g2", torch.sigmoid, self.res_gate2)
        x = torch.addcmul(x, g1, mo)
        return torch.addcmul(x, g2, self.ffn(self.norm2(x)))

    def forward(self, x, state=None, conv_state=None, past_c_kv=None):
        h = self.norm1(x)
        if self.is_attention:
            mo, nc = self.mixer(h, past_c_kv=past_c_kv)
            return self._residual(x, mo), None, None, nc
        mo, ns, ncv = self.mixer(h, state=state, conv_state=conv_state)
        return self._residual(x, mo), ns, ncv, None

    def step(self, x, state=None, conv_state=None, past_c_kv=None):
        h = self.norm1(x)
        if self.is_attention:
            mo, nc = self.mixer(h, past_c_kv=past_c_kv)
            return self._residual(x, mo), None, None, nc
        mo, ns, ncv = self.mixer.step(h, state=state, conv_state=conv_state)
        return self._residual(x, mo), ns, ncv, None

    def decode(self, x, state=None, conv_state=None, cache: Optional[LatentCache] = None):
        """One token: DGDA blocks carry (state, conv_state); MABA-SA blocks append to and
        decode over ``cache``."""
        h = self.norm1(x)
        if self.is_attention:
            return self._residual(x, self.mixer.decode_step(h, cache)), None, None
        mo, ns, ncv = self.mixer.step(h, state=state, conv_state=conv_state)
        return self._residual(x, mo), ns, ncv


class ServingStep:
    """Device-resident state of a greedy decode after a prefill, and one decode token over it.

    Everything a step reads or writes sits in buffers that keep their addresses: the current
    token, a device counter pair ``[n, n + 1]`` (rows held before the step and after it), the
    DGDA states and conv histories (updated in place), and per MABA-SA block a
    ``DeviceCache`` (appended on device).  So the step can be captured once as a HIP graph
    and replayed for every position.  The residual stream runs through the fused HIP kernels:
    gated residual + the next RMSNorm in one launch, SwiGLU's activation in one launch."""

    def __init__(self, model: "MabaSparseForCausalLM", states, length: int, capacity: int,
                 first_token: torch.Tensor) -> None:
        self.model = model
        dev = first_token.device
        self.tok = first_token.clone()
        self.counters = torch.tensor([length, length + 1], dtype=torch.long, device=dev)
        self.capacity = capacity
        self.dgda, self.caches = {}, {}
        for i, (layer, (st, cv, ck)) in enumerate(zip(model.layers, states)):
            if layer.is_attention:
                keys = layer.mixer.indexer._cached_k_idx
                self.caches[i] = DeviceCache(ck, keys, capacity, pool=layer.mixer.hca_pool_size,
                                             block=layer.mixer.block_size)
            else:
                self.dgda[i] = (st.clone().contiguous(), [h.clone().contiguous() for h in cv])
        self.last: Optional[torch.Tensor] = None
        self.decode_linear = ServingStep.decode_linear and _decode_linear_fits(model)

    # every linear layer of a step as a HIP decode linear that builds its input in the same
    # launch (see step); False keeps torch's GEMMs and the separate norm / SwiGLU kernels
    decode_linear = True

    def step(self) -> None:
        """Decode the token in ``tok``; leaves the next token in ``tok`` and its logits in ``last``.

        With ``decode_linear`` each linear layer is one HIP launch that also makes its input:
        the embedding projection gathers the token's table rows, the mixer's first projection
        normalises the layer input and, from the second layer on,
        first adds the previous FFN output through the gated residual (writing the new residual
        stream to a fresh buffer); the stacked gate/up projection does the same for the
        mixer's output; the down projection applies SwiGLU's activation; and the head
        projection takes the last residual through the final norm; the greedy pick is one
        HIP argmax launch."""
        if self.decode_linear:
            return self._step_decode_linear()
        from maba_sparse.kernels import hip_backend as hb
        m = self.model
        layers = m.layers
        x = m.embeddings(self.tok)
        n1 = layers[0].norm1
        h = hb.hip_rmsnorm(x, n1.weight, n1.eps)
        for i, layer in enumerate(layers):
            if layer.is_attention:
                mo = layer.mixer.decode_step_device(h, self.caches[i], self.counters)
            else:
                st, hs = self.dgda[i]
                mo = layer.mixer.step_device(h, st, hs)
            g1 = _frozen(layer, "g1", torch.sigmoid, layer.res_gate1)
            g2 = _frozen(layer, "g2", torch.sigmoid, layer.res_gate2)
            h2 = hb.hip_rmsnorm(x, layer.norm2.weight, layer.norm2.eps, mo=mo, gate=g1, x_out=x)
            f = layer.ffn.forward_hip(h2)
            nxt = layers[i + 1].norm1 if i + 1 < len(layers) else m.final_norm
            h = hb.hip_rmsnorm(x, nxt.weight, nxt.eps, mo=f, gate=g2, x_out=x)
        self.last = m.lm_head(m.head_proj(h))[:, -1]
        self.tok.copy_(self.last.argmax(dim=-1, keepdim=True))
        self.counters += 1

    def _step_decode_linear(self) -> None:
        from maba_sparse.kernels import hip_backend as hb
        m = self.model
        layers = m.layers
        emb = m.embeddings
        x = hb.hip_decode_linear(emb.in_emb.weight, emb.proj.weight, rows=self.tok)
        n1 = layers[0].norm1
        spec = dict(a=x, norm_w=n1.weight, eps=n1.eps)    # the input stage of the next projection
        for i, layer in enumerate(layers):
            def proj(w, spec=spec):
                return hb.hip_decode_linear(weight=w, **spec)
            if layer.is_attention:
                mo = layer.mixer.decode_step_device(x, self.caches[i], self.counters, proj=proj)
            else:
                st, hs = self.dgda[i]
                mo = layer.mixer.step_device(x, st, hs, proj=proj)
            x = spec.get("x_out", x)                     # the residual stream after that stage
            g1 = _frozen(layer, "g1", torch.sigmoid, layer.res_gate1)
            g2 = _frozen(layer, "g2", torch.sigmoid, layer.res_gate2)
            ffn = layer.ffn
            w_gu = _frozen(ffn, "gate_up", lambda a, b: torch.cat([a, b], dim=0), ffn.w_gate.weight, ffn.w_up.weight)
            x2 = torch.empty_like(x)
            gu = hb.hip_decode_linear(x, w_gu, norm_w=layer.norm2.weight, eps=layer.norm2.eps, mo=mo, gate=g1,
                                      x_out=x2)
            f = hb.hip_decode_linear(gu, ffn.w_down.weight, swiglu=True)
            x = x2
            nxt = layers[i + 1].norm1 if i + 1 < len(layers) else m.final_norm
            spec = dict(a=x, norm_w=nxt.weight, eps=nxt.eps, mo=f, gate=g2, x_out=torch.empty_like(x))
        hp = hb.hip_decode_linear(weight=m.head_proj.weight, **spec)
        logits = hb.hip_decode_linear(hp, m.lm_head.weight)
        self.last = logits[:, -1]
        hb.hip_argmax_rows(logits, out=self.tok)
        self.counters += 1


def _decode_linear_fits(model: "MabaSparseForCausalLM") -> bool:
    """Whether every linear layer of a serving step fits the HIP decode linear: bf16 weights
    (and embedding table), no bias (the MABA-SA stream gate's is added after the stacked
    projection), input widths a multiple of 32, at most 2048 where the input is normalised and
    4096 elsewhere; bf16 norm weights and residual gates; a vocabulary of whole 8-wide vectors
    for the argmax."""
    normed, plain = [model.head_proj], [model.embeddings.in_emb, model.embeddings.proj, model.lm_head]
    if model.config.vocab_size % 8:
        return False                                       # the argmax kernel's row vectors
    for layer in model.layers:
        mx = layer.mixer
        normed += [layer.ffn.w_gate, layer.ffn.w_up]
        plain += [layer.ffn.w_down, mx.o_proj]
        if layer.is_attention:
            normed += [mx.indexer.q_idx_proj, mx.indexer.k_idx_proj, mx.q_proj, mx.kv_down_proj]
            if mx.stream_gate.weight.shape[1] % 32 or mx.stream_gate.weight.dtype != torch.bfloat16:
                return False
        else:
            normed += [mx.q_proj, mx.k_proj, mx.v_proj, mx.gate_alpha, mx.gate_erase, mx.gate_write]
    for lim, mods in ((2048, normed), (4096, plain)):
        for mod in mods:
            w = mod.weight
            if (w.dtype != torch.bfloat16 or w.dim() != 2 or w.shape[1] % 32 or w.shape[1] > lim
                    or getattr(mod, "bias", None) is not None):
                return False
    vecs = [model.final_norm.weight] + [t for l in model.layers
                                        for t in (l.norm1.weight, l.norm2.weight, l.res_gate1, l.res_gate2)]
    return all(t.dtype == torch.bfloat16 for t in vecs)


class MabaSparseForCausalLM(WeightCacheMixin, nn.Module):
    def __init__(self, config: Optional[MabaConfig] = None) -> None:
        super().__init__()
        self.config = config or get_101m_config()
        c = self.config
        self.embeddings = FactorizedEmbeddings(c.vocab_size, c.d_emb, c.dim)
        self.layers = nn.ModuleList([MabaBlock(c, i) for i in range(c.n_layers)])
        self.final_norm = RMSNorm(c.dim, eps=c.rms_norm_eps)
        self.head_proj = nn.Linear(c.dim, c.d_emb, bias=False)
        self.lm_head = nn.Linear(c.d_emb, c.vocab_size, bias=False)
        self.lm_head.weight = self.embeddings.in_emb.weight      # tied (model.py:205)
        self._install_weight_cache_hooks()

    def init_normal(self, std: float = 0.02) -> "MabaSparseForCausalLM":
        """Every weight matrix and embedding ~ N(0, std) (the BASELINE's random init); norms,
        biases and residual gates keep their constructor values."""
        with torch.no_grad():
            for m in self.modules():
                if isinstance(m, (nn.Linear, nn.Embedding)):
                    m.weight.normal_(0.0, std)
        return self

    def _logits(self, x: torch.Tensor) -> torch.Tensor:
        return self.lm_head(self.head_proj(self.final_norm(x)))

    def forward(self, input_ids: torch.Tensor, past_states: Optional[List[Any]] = None, last_only: bool = False):
        """Prefill: ``(logits, past_states)`` with ``(state, conv_state, c_kv)`` per block
        (reference model.py:207-234; the loss and MTP head are left out).  ``last_only`` returns
        the logits of the last position only, ``[B, 1, vocab]`` (what generation reads)."""
        x = self.embeddings(input_ids)
        if self._fused_norms_ok(x):
            return self._forward_fused_norms(x, past_states, last_only)
        nps = []
        for i, layer in enumerate(self.layers):
            st, cv, pk = past_states[i] if past_states is not None else (None, None, None)
            x, nst, ncv, nck = layer(x, state=st, conv_state=cv, past_c_kv=pk)
            nps.append((nst, ncv, nck))
        return self._logits(x[:, -1:] if last_only else x), nps

    def _fused_norms_ok(self, x: torch.Tensor) -> bool:
        """Whether ``forward`` runs its norms, gated residuals and SwiGLU activations as HIP
        kernels: the ``hip`` backend, a bf16 model, the kernels' widths, no gradients."""
        c = self.config
        if x.device.type != "cuda" or get_backend(x.device) != "hip" or x.dtype != torch.bfloat16:
            return False
        if c.dim % 2 or c.dim > 2048 or c.intermediate_size % 2:
            return False
        return not (torch.is_grad_enabled() and any(p.requires_grad for p in self.parameters()))

    def _forward_fused_norms(self, x: torch.Tensor, past_states, last_only: bool = False):
        """``forward`` with each block's ``x + g1 * mo`` and ``RMSNorm`` in one HIP launch, its
        ``x + g2 * ffn`` folded into the next block's (or the final) norm, and the SwiGLU
        activation as one kernel (the block structure of model.py:92-128; the mixers as in
        ``MabaBlock.forward``).  The residual stream is updated in place in ``x``."""
        from maba_sparse.kernels import hip_backend as hb
        layers = self.layers
        n1 = layers[0].norm1
        h = hb.hip_rmsnorm(x, n1.weight, n1.eps)
        nps = []
        for i, layer in enumerate(layers):
            st, cv, pk = past_states[i] if past_states is not None else (None, None, None)
            nst = ncv = nck = None
            if layer.is_attention:
                mo, nck = layer.mixer(h, past_c_kv=pk)
            else:
                mo, nst, ncv = layer.mixer(h, state=st, conv_state=cv)
            g1 = _frozen(layer, "g1", torch.sigmoid, layer.res_gate1)
            g2 = _frozen(layer, "g2", torch.sigmoid, layer.res_gate2)
            h2 = hb.hip_rmsnorm(x, layer.norm2.weight, layer.norm2.eps, mo=mo, gate=g1, x_out=x)
            f = layer.ffn.forward_hip(h2)
            nxt = layers[i + 1].norm1 if i + 1 < len(layers) else self.final_norm
            h = hb.hip_rmsnorm(x, nxt.weight, nxt.eps, mo=f, gate=g2, x_out=x)
            nps.append((nst, ncv, nck))
        return self.lm_head(self.head_proj(h[:, -1:] if last_only else h)), nps

    def step(self, input_ids: torch.Tensor, past_states: Optional[List[Any]] = None):
        """One token with the reference's state passing (model.py:251-270)."""
        if input_ids.shape[1] != 1:
            raise ValueError(f"step() expects single-token input (L=1), got L={input_ids.shape[1]}")
        x = self.embeddings(input_ids)
        nps = []
        for i, layer in enumerate(self.layers):
            st, cv, pk = past_states[i] if past_states is not None else (None, None, None)
            x, nst, ncv, nck = layer.step(x, state=st, conv_state=cv, past_c_kv=pk)
            nps.append((nst, ncv, nck))
        return self._logits(x), nps

    def serving_graph_ok(self, input_ids: torch.Tensor) -> bool:
        """Whether ``generate_greedy`` can take the captured device-resident step: the HIP
        backend, a bf16 model, and a prefill holding at least ``top_k`` blocks (the decode
        indexer then always selects ``top_k`` of them)."""
        c = self.config
        if input_ids.device.type != "cuda" or get_backend(input_ids.device) != "hip":
            return False
        if next(self.parameters()).dtype != torch.bfloat16:
            return False
        if c.dim % 2 or c.dim > 2048 or c.intermediate_size % 2:       # the fused norm and SwiGLU kernels
            return False
        for layer in self.layers:
            mx = layer.mixer
            if layer.is_attention:
                if mx.d_c % 32 or mx.d_c > 128 or mx.indexer.d_idx % 32 or mx.indexer.d_idx > 256:
                    return False
                if mx.n_heads > 16 or mx.top_k > 64 or mx.block_size > 64:
                    return False
            elif mx.d_k != 64 or mx.d_v != 64 or mx.kernel_size != 4 or mx.n_heads > 16:
                return False
        return input_ids.shape[1] >= c.top_k * c.block_size

    @torch.no_grad()
    def generate_greedy(self, input_ids: torch.Tensor, max_new_tokens: int,
                        on_prefill_done=None, return_logits: bool = False, graph: Optional[bool] = None,
                        on_graph_ready=None):
        """Greedy decoding (reference model.py:272-305 at temperature 0): one prefill, then
        ``max_new_tokens - 1`` single-token steps over per-layer decode caches.  Returns the
        new tokens ``[B, max_new_tokens]``.  ``on_prefill_done()`` runs between the two phases
        and ``on_graph_ready()`` (graph path) once the step graph is captured, before its first
        replay (timing hooks).  With ``return_logits`` the last-position logits of the prefill and
        of every step come back too, ``[B, max_new_tokens, vocab]``.

        ``graph`` (default: whenever ``serving_graph_ok``) takes the device-resident path: a
        ``ServingStep`` whose first step runs eagerly (it also warms up the libraries), then
        one HIP graph of a step, captured once and replayed for every further token.
        Otherwise each step runs eagerly over ``LatentCache``s.

        The stacked and converted weights the decode path keeps are dropped on entry, so a
        weight written through ``.data`` since the last call takes effect."""
        self.clear_weight_caches()
        B, L = input_ids.shape
        if graph is None:
            graph = self.serving_graph_ok(input_ids)
        logits, states = self(input_ids, last_only=True)
        if graph:
            return self._generate_graph(logits, states, L, max_new_tokens, on_prefill_done, return_logits,
                                        on_graph_ready)
        caches: List[Optional[LatentCache]] = []
        for layer, (_, _, c_kv) in zip(self.layers, states):
            if layer.is_attention:
                cache = LatentCache(B, L + max_new_tokens, self.config.d_c, pool=self.config.hca_pool_size,
                                    device=input_ids.device, dtype=c_kv.dtype)
                cache.append(c_kv)
                caches.append(cache)
            else:
                caches.append(None)
        if on_prefill_done is not None:
            on_prefill_done()
        last = logits[:, -1]
        tok = last.argmax(dim=-1, keepdim=True)
        out = [tok]
        seen = [last] if return_logits else None
        for _ in range(max_new_tokens - 1):
            x = self.embeddings(tok)
            for i, layer in enumerate(self.layers):
                st, cv, _ = states[i]
                x, nst, ncv = layer.decode(x, state=st, conv_state=cv, cache=caches[i])
                states[i] = (nst, ncv, None)
            last = self._logits(x)[:, -1]
            tok = last.argmax(dim=-1, keepdim=True)
            out.append(tok)
            if return_logits:
                seen.append(last)
        toks = torch.cat(out, dim=1)
        return (toks, torch.stack(seen, dim=1)) if return_logits else toks

    def _generate_graph(self, logits, states, L, max_new_tokens, on_prefill_done, return_logits,
                        on_graph_ready=None):
        last = logits[:, -1]
        first = last.argmax(dim=-1, keepdim=True)
        serv = ServingStep(self, states, L, L + max_new_tokens, first)
        del states
        if on_prefill_done is not None:
            on_prefill_done()
        out, seen = [first], ([last] if return_logits else None)

        def keep():
            out.append(serv.tok.clone())
            if return_logits:
                seen.append(serv.last.clone())

        steps = max_new_tokens - 1
        if steps > 0:
            side = torch.cuda.Stream(device=first.device)
            side.wait_stream(torch.cuda.current_stream(first.device))
            with torch.cuda.stream(side):      # the first step, eager: lazy library set-up happens here
                serv.step()
            torch.cuda.current_stream(first.device).wait_stream(side)
            keep()
        if steps > 1:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):          # recorded, not run
                serv.step()
            if on_graph_ready is not None:
                on_graph_ready()
            for _ in range(steps - 1):
                g.replay()
                keep()
        toks = torch.cat(out, dim=1)
        return (toks, torch.stack(seen, dim=1)) if return_logits else toks


MabaSparseLM = MabaSparseForCausalLM
MabaLM = MabaSparseForCausalLM
