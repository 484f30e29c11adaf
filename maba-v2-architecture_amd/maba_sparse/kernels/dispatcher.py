"""Kernel registry and dispatcher -- the drop-in boundary of the hot path.

Mirrors the public contract of the reference dispatcher
(``maba_sparse/kernels/dispatcher.py``): the registry and ``register_kernel`` /
``get_kernel`` (:31-111), ``get_backend`` routing with the ``MABA_BACKEND``
override (:181-238), the five ``dispatch_*`` ops with keyword-only kernel
calls (:258-508) and the once-per-``backend:op`` fallback warning with
``MABA_STRICT_BACKEND`` escalation (:241-255).

Differences, all deliberate:

* The GPU backend is ``"hip"`` (gfx950 kernels in ``libmaba_hip.so``).  A ROCm
  GPU tensor routes to it; ``MABA_BACKEND=hip`` selects it and the reference's
  GPU names ``triton``/``cuda``/``gpu`` map to it.  ``rocm`` stays invalid, as
  the reference's tests require.
* A missing HIP library is never papered over: ``HipLibraryMissing`` propagates
  instead of falling back, so a GPU run cannot silently take a non-HIP path.
* Five ops the reference only has as inline torch code get dispatcher entries:
  ``index_topk_decode`` (layers/indexer.py:101-112), ``hca_pool``
  (layers/sparse_attention.py:206), ``maba_sa_decode``
  (layers/sparse_attention.py:79-219,263-275), ``maba_sa_prefill`` (the three
  prefill streams and their gate, layers/sparse_attention.py:95-219,275) and
  ``dgda_prologue`` (the DGDA layer's conv, gates and key normalisation,
  layers/dgda.py:103-121,186-207).
* ``allow_mixed_dtypes=True`` (keyword) lets ``dgda_prefill``/``dgda_step``
  accept bf16 q/k/v with fp32 gates and state; without it the reference's
  "dtypes must match" ``TypeError`` is kept.
"""
from __future__ import annotations

import logging
import os
import warnings
from typing import Any, Callable, Dict, Optional, Set, Tuple, Union

import torch

from maba_sparse._native import HipLibraryMissing
from maba_sparse.kernels import common as _c
from maba_sparse.kernels import cpu_dgda as _cpu

logger = logging.getLogger(__name__)

_KERNEL_REGISTRY: Dict[str, Dict[str, Callable]] = {
    "reference": {
        "dgda_prefill": _c.reference_dgda_prefill,
        "dgda_step": _c.reference_dgda_step,
        "compute_centroids": _c.reference_compute_centroids,
        "index_topk": _c.reference_index_topk,
        "stream_superposition": _c.reference_stream_superposition,
        "index_topk_decode": _c.ref_index_topk_decode,
        "hca_pool": _c.ref_hca_pool,
        "maba_sa_decode": _c.ref_maba_sa_decode,
        "dgda_prologue": _c.ref_dgda_prologue,
        "maba_sa_prefill": _c.ref_maba_sa_prefill,
    },
    # host cores: the chunked DGDA of the reference's CPU backend (cpu_dgda.py), the rest as
    # the reference ops in torch
    "cpu": {
        "dgda_prefill": _cpu.cpu_dgda_prefill,
        "dgda_step": _cpu.cpu_dgda_step,
        "compute_centroids": _c.reference_compute_centroids,
        "index_topk": _c.reference_index_topk,
        "stream_superposition": _c.reference_stream_superposition,
        "index_topk_decode": _c.ref_index_topk_decode,
        "hca_pool": _c.ref_hca_pool,
        "maba_sa_decode": _c.ref_maba_sa_decode,
        "dgda_prologue": _c.ref_dgda_prologue,
        "maba_sa_prefill": _c.ref_maba_sa_prefill,
    },
    "hip": {},
    "xla": {},
}

_WARNED_FALLBACKS: Set[str] = set()
_BACKEND_CACHE: Dict[Tuple[Optional[str], Optional[int], Optional[str]], str] = {}
_HIP_IMPORTED = False


def clear_dispatcher_cache() -> None:
    _BACKEND_CACHE.clear()


def clear_fallback_warnings() -> None:
    _WARNED_FALLBACKS.clear()
    clear_dispatcher_cache()


def register_kernel(backend: str, op_name: str) -> Callable:
    """Decorator registering ``fn`` as ``op_name`` of ``backend`` (creates both on demand)."""
    def decorator(fn: Callable) -> Callable:
        _KERNEL_REGISTRY.setdefault(backend, {})[op_name] = fn
        return fn
    return decorator


def _ensure_hip_registered() -> None:
    global _HIP_IMPORTED
    if not _HIP_IMPORTED:
        _HIP_IMPORTED = True
        import maba_sparse.kernels.hip_backend  # noqa: F401  (registers on import)


def get_kernel(backend: str, op_name: str) -> Optional[Callable]:
    if backend == "hip":
        _ensure_hip_registered()
    return _KERNEL_REGISTRY.get(backend, {}).get(op_name)


def is_rocm_gpu_available(device: Optional[Union[torch.device, str, int]] = None) -> bool:
    """True when torch is a ROCm build and a GPU is visible."""
    return bool(getattr(torch.version, "hip", None)) and torch.cuda.is_available()


def is_hip_backend_available() -> bool:
    from maba_sparse import _native
    return _native.available()


def is_openmp_available() -> bool:
    try:
        return bool(torch.backends.openmp.is_available())
    except Exception:
        return False


def _parse_device(device) -> Tuple[Optional[str], Optional[int]]:
    if device is None:
        return None, None
    if isinstance(device, int):
        return "cuda", device
    d = torch.device(device) if isinstance(device, str) else device
    return d.type, (d.index if d.index is not None else 0)


def get_backend(device: Union[torch.device, str, None] = None) -> str:
    """Backend name for ``device`` (reference dispatcher.py:181-238, with ``hip``)."""
    try:
        dev_type, dev_idx = _parse_device(device)
    except Exception:
        return "reference"
    env = os.environ.get("MABA_BACKEND")
    key = (dev_type, dev_idx, env)
    hit = _BACKEND_CACHE.get(key)
    if hit is not None:
        return hit
    if env and env.lower() != "auto":
        val = env.lower()
        if val in ("hip", "triton", "cuda", "gpu"):
            res = "hip"
        elif val in ("xla", "tpu"):
            res = "xla"
        elif val in ("cpu", "openmp"):
            res = "cpu"
        elif val in ("reference", "pytorch", "ref"):
            res = "reference"
        else:
            raise ValueError(
                f"Unsupported MABA_BACKEND '{env}'. Supported: ['auto', 'hip', 'triton', 'cpu', 'xla', "
                f"'reference', 'ref']"
            )
    elif dev_type is None:
        res = "hip" if is_rocm_gpu_available() else "cpu"
    elif dev_type == "cuda":
        res = "hip" if getattr(torch.version, "hip", None) else "reference"
    elif dev_type == "cpu":
        res = "cpu"
    else:
        res = "reference"
    _BACKEND_CACHE[key] = res
    return res


def _log_fallback_warning(op_name: str, backend: str, exc: Optional[Exception] = None) -> None:
    strict = os.environ.get("MABA_STRICT_BACKEND", "0").lower() in ("1", "true")
    detail = f" ({type(exc).__name__}: {exc})" if exc is not None else ""
    msg = (f"[Maba Dispatcher Fallback] Native kernel for '{op_name}' on backend '{backend}' "
           f"is unavailable or failed{detail}. Falling back to reference.")
    if strict:
        raise RuntimeError(msg)
    key = f"{backend}:{op_name}"
    if key not in _WARNED_FALLBACKS:
        _WARNED_FALLBACKS.add(key)
        warnings.warn(msg, RuntimeWarning, stacklevel=3)
        logger.debug(msg)


def _run(op_name: str, device, kwargs: Dict[str, Any]):
    backend = get_backend(device)
    fn = get_kernel(backend, op_name)
    if fn is not None and backend != "reference":
        try:
            return fn(**kwargs)
        except HipLibraryMissing:
            raise
        except Exception as exc:
            _log_fallback_warning(op_name, backend, exc)
    elif backend != "reference" and fn is None:
        _log_fallback_warning(op_name, backend, None)
    ref = get_kernel("reference", op_name)
    kwargs = {k: v for k, v in kwargs.items() if k != "allow_mixed_dtypes"}
    return ref(**kwargs)


def _dgda_precheck(q, k, v, alpha, b, w, log_alpha, extra_name, extra, mixed: bool) -> None:
    """Cheap checks the reference dispatcher runs before routing (dispatcher.py:270-305)."""
    if alpha is None and log_alpha is None:
        raise ValueError("Either alpha or log_alpha must be provided")
    if b is None or w is None:
        raise ValueError("Both b and w gate tensors must be provided")
    if q.dtype not in (torch.float32, torch.float16, torch.bfloat16, torch.float64):
        raise TypeError(f"Unsupported dtype {q.dtype}. Supported: "
                        f"{(torch.float32, torch.float16, torch.bfloat16, torch.float64)}")
    named = [("k", k), ("v", v), ("b", b), ("w", w), ("alpha", alpha), ("log_alpha", log_alpha),
             (extra_name, extra)]
    for name, t in named:
        if t is None:
            continue
        if t.device != q.device:
            raise RuntimeError(
                f"Expected all tensors to be on the same device, but got {q.device} and {t.device} for {name}")
        if not mixed and t.dtype != q.dtype:
            raise TypeError(f"Tensor dtypes must match, but got {q.dtype} for q and {t.dtype} for {name}")


def dispatch_dgda_prefill(q, k, v, alpha=None, b=None, w=None, chunk_size: int = 16, initial_state=None,
                          log_alpha=None, **kwargs: Any) -> Tuple[torch.Tensor, torch.Tensor]:
    _dgda_precheck(q, k, v, alpha, b, w, log_alpha, "initial_state", initial_state,
                   bool(kwargs.get("allow_mixed_dtypes", False)))
    return _run("dgda_prefill", q.device, dict(q=q, k=k, v=v, alpha=alpha, b=b, w=w, chunk_size=chunk_size,
                                               initial_state=initial_state, log_alpha=log_alpha, **kwargs))


def dispatch_dgda_step(q, k, v, alpha=None, b=None, w=None, state=None, log_alpha=None,
                       **kwargs: Any) -> Tuple[torch.Tensor, torch.Tensor]:
    _dgda_precheck(q, k, v, alpha, b, w, log_alpha, "state", state,
                   bool(kwargs.get("allow_mixed_dtypes", False)))
    return _run("dgda_step", q.device, dict(q=q, k=k, v=v, alpha=alpha, b=b, w=w, state=state,
                                            log_alpha=log_alpha, **kwargs))


def dispatch_compute_centroids(k_idx, block_size: int = 64, **kwargs: Any) -> torch.Tensor:
    _c.validate_indexer_inputs(k_idx=k_idx)
    if block_size <= 0:
        raise ValueError(f"block_size must be positive, got {block_size}")
    return _run("compute_centroids", k_idx.device, dict(k_idx=k_idx, block_size=block_size, **kwargs))


def dispatch_index_topk(q_idx, centroids, lambda_dist: float = 0.5, top_k: int = 32, block_size: int = 64,
                        **kwargs: Any):
    if q_idx.device != centroids.device:
        raise RuntimeError(
            f"Expected all tensors to be on the same device, but got {q_idx.device} and {centroids.device}")
    if q_idx.dim() != 3 or centroids.dim() != 3:
        raise ValueError(f"q_idx and centroids must be 3D, got {q_idx.dim()}D and {centroids.dim()}D")
    if q_idx.shape[0] != centroids.shape[0] or q_idx.shape[2] != centroids.shape[2]:
        raise ValueError(
            f"Dimension mismatch between q_idx {list(q_idx.shape)} and centroids {list(centroids.shape)}")
    if top_k <= 0:
        raise ValueError(f"top_k must be positive, got {top_k}")
    if block_size <= 0:
        raise ValueError(f"block_size must be positive, got {block_size}")
    return _run("index_topk", q_idx.device, dict(q_idx=q_idx, centroids=centroids, lambda_dist=lambda_dist,
                                                 top_k=top_k, block_size=block_size, **kwargs))


def dispatch_index_topk_decode(q, centroids, lambda_dist: float = 0.5, top_k: int = 32, **kwargs: Any):
    """Decode-step scoring + top-k; ``q [B, Hq, d]``, ``centroids [B, nb, d]``."""
    if q.device != centroids.device:
        raise RuntimeError(
            f"Expected all tensors to be on the same device, but got {q.device} and {centroids.device}")
    if q.dim() != 3 or centroids.dim() != 3 or q.shape[0] != centroids.shape[0] or q.shape[2] != centroids.shape[2]:
        raise ValueError(f"Dimension mismatch between q {list(q.shape)} and centroids {list(centroids.shape)}")
    if top_k <= 0:
        raise ValueError(f"top_k must be positive, got {top_k}")
    return _run("index_topk_decode", q.device, dict(q=q, centroids=centroids, lambda_dist=lambda_dist,
                                                    top_k=top_k, **kwargs))


def dispatch_stream_superposition(o_local, o_sparse, o_hca, gate_logits=None, **kwargs: Any) -> torch.Tensor:
    dev = o_local.device
    if o_sparse.device != dev or o_hca.device != dev:
        raise RuntimeError(
            f"Expected all tensors to be on the same device, but got {dev}, {o_sparse.device}, {o_hca.device}")
    gate = gate_logits if gate_logits is not None else kwargs.get("gate_weights")
    if gate is not None and gate.device != dev:
        raise RuntimeError(f"Expected all tensors to be on the same device, but got {dev} and {gate.device}")
    _c.validate_superposition_inputs(o_local, o_sparse, o_hca, gate)
    return _run("stream_superposition", dev, dict(o_local=o_local, o_sparse=o_sparse, o_hca=o_hca,
                                                  gate_logits=gate_logits, **kwargs))


def dispatch_hca_pool(c_kv, pool: int = 64, **kwargs: Any) -> torch.Tensor:
    if c_kv.dim() != 3:
        raise ValueError(f"c_kv must be 3D [B, L, d_c], got {list(c_kv.shape)}")
    if pool <= 0:
        raise ValueError(f"pool must be positive, got {pool}")
    return _run("hca_pool", c_kv.device, dict(c_kv=c_kv, pool=pool, **kwargs))


def dispatch_maba_sa_decode(q_lat, c_kv, hca, idx, gate, L: int, scale: float, window: int = 128,
                            n_sink: int = 4, block_size: int = 64, pool: int = 64, **kwargs: Any) -> torch.Tensor:
    """Fused three-stream MABA-SA decode in latent space (see ``common.ref_maba_sa_decode``)."""
    for name, t in (("c_kv", c_kv), ("hca", hca), ("idx", idx), ("gate", gate)):
        if t.device != q_lat.device:
            raise RuntimeError(
                f"Expected all tensors to be on the same device, but got {q_lat.device} and {t.device} for {name}")
    if L <= 0 or L > c_kv.shape[1]:
        raise ValueError(f"L={L} must be in [1, {c_kv.shape[1]}]")
    return _run("maba_sa_decode", q_lat.device, dict(q_lat=q_lat, c_kv=c_kv, hca=hca, idx=idx, gate=gate, L=L,
                                                     scale=scale, window=window, n_sink=n_sink,
                                                     block_size=block_size, pool=pool, **kwargs))


def dispatch_dgda_prologue(projections, conv_weights, history=None, n_heads: int = 10, eps: float = 1e-6,
                           gate_dtype: Optional[torch.dtype] = None, with_alpha: bool = True, **kwargs: Any):
    """The DGDA layer's op inputs from its six projections (see ``common.ref_dgda_prologue``)."""
    if len(projections) != 6 or len(conv_weights) != 3 or (history is not None and len(history) != 3):
        raise ValueError("dgda_prologue takes six projections, three conv weights and three histories or None")
    dev = projections[0].device
    for t in (*projections, *conv_weights, *(history or ())):
        if t.device != dev:
            raise RuntimeError(f"Expected all tensors to be on the same device, but got {dev} and {t.device}")
    shape = projections[0].shape
    if len(shape) != 3 or any(p.shape != shape for p in projections):
        raise ValueError(f"projections must share one [B, L, C] shape, got {[list(p.shape) for p in projections]}")
    if shape[2] % n_heads != 0:
        raise ValueError(f"C={shape[2]} is not a multiple of n_heads={n_heads}")
    return _run("dgda_prologue", dev, dict(projections=projections, conv_weights=conv_weights, history=history,
                                           n_heads=n_heads, eps=eps, gate_dtype=gate_dtype, with_alpha=with_alpha,
                                           **kwargs))


def dispatch_maba_sa_prefill(q, k, v, kh, vh, early, idx, gate_logits, scale: float, window: int = 128,
                             n_sink: int = 4, block_size: int = 64, pool: int = 64, **kwargs: Any) -> torch.Tensor:
    """The three MABA-SA prefill streams and their gate (see ``common.ref_maba_sa_prefill``)."""
    dev = q.device
    for name, t in (("k", k), ("v", v), ("kh", kh), ("vh", vh), ("early", early), ("idx", idx),
                    ("gate_logits", gate_logits)):
        if t is not None and t.device != dev:
            raise RuntimeError(f"Expected all tensors to be on the same device, but got {dev} and {t.device} for {name}")
    if q.dim() != 4 or k.dim() != 4 or v.shape != k.shape or q.shape[:2] != k.shape[:2] or q.shape[3] != k.shape[3]:
        raise ValueError(f"q [B,H,Lq,dh] and k, v [B,H,Lkv,dh] expected, got {list(q.shape)}, {list(k.shape)}")
    if q.shape[2] > k.shape[2]:
        raise ValueError(f"more queries ({q.shape[2]}) than keys ({k.shape[2]})")
    return _run("maba_sa_prefill", dev, dict(q=q, k=k, v=v, kh=kh, vh=vh, early=early, idx=idx,
                                             gate_logits=gate_logits, scale=scale, window=window, n_sink=n_sink,
                                             block_size=block_size, pool=pool, **kwargs))


dgda_prefill = dispatch_dgda_prefill
dgda_step = dispatch_dgda_step
compute_centroids = dispatch_compute_centroids
index_topk = dispatch_index_topk
stream_superposition = dispatch_stream_superposition
index_topk_decode = dispatch_index_topk_decode
hca_pool = dispatch_hca_pool
maba_sa_decode = dispatch_maba_sa_decode
dgda_prologue = dispatch_dgda_prologue
maba_sa_prefill = dispatch_maba_sa_prefill
ref_dgda_prefill = _c.ref_dgda_prefill
ref_dgda_step = _c.ref_dgda_step
ref_centroids = _c.ref_centroids
ref_topk = _c.ref_topk
ref_superposition = _c.ref_superposition
