"""ctypes binding of ``libmaba_hip.so`` (the gfx950 HIP kernels behind ``include/maba_hip.h``).

The library is built in-tree by ``__graft_entry__.build()`` (or
``python -m maba_sparse.build``) into ``maba_sparse/_lib/libmaba_hip.so``.  This
module never compiles anything; a missing library raises ``HipLibraryMissing``
when a HIP op is called, so a GPU run can never silently take another path.
"""
from __future__ import annotations

import ctypes
import os
import struct
import threading
from typing import Optional, Sequence

import torch

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib")
# MABA_HIP_LIBRARY names another build of the same library (a missing file still raises)
LIB_PATH = os.environ.get("MABA_HIP_LIBRARY") or os.path.join(LIB_DIR, "libmaba_hip.so")

MABA_F32, MABA_F16, MABA_BF16, MABA_F64, MABA_I64, MABA_I32 = 0, 1, 2, 3, 4, 5
_DTYPE_CODES = {
    torch.float32: MABA_F32,
    torch.float16: MABA_F16,
    torch.bfloat16: MABA_BF16,
    torch.float64: MABA_F64,
    torch.int64: MABA_I64,
    torch.int32: MABA_I32,
}

MABA_OK, MABA_ERR_INVALID, MABA_ERR_DTYPE, MABA_ERR_UNSUPPORTED, MABA_ERR_HIP, MABA_ERR_WORKSPACE = range(6)

# Every symbol declared in include/maba_hip.h.
EXPORTED_SYMBOLS = (
    "maba_hip_last_error",
    "maba_hip_abi_version",
    "maba_hip_dgda_prefill_workspace_size",
    "maba_hip_dgda_prefill",
    "maba_hip_dgda_step",
    "maba_hip_compute_centroids",
    "maba_hip_index_topk",
    "maba_hip_index_topk_decode_workspace_size",
    "maba_hip_index_topk_decode",
    "maba_hip_stream_superposition",
    "maba_hip_hca_pool",
    "maba_hip_maba_sa_decode_workspace_size",
    "maba_hip_maba_sa_decode",
    "maba_hip_maba_sa_decode_static",
    "maba_hip_dgda_prologue",
    "maba_hip_maba_sa_prefill",
    "maba_hip_cache_append",
    "maba_hip_index_topk_decode_dev",
    "maba_hip_maba_sa_decode_dev",
    "maba_hip_rmsnorm",
    "maba_hip_swiglu",
    "maba_hip_maba_sa_prefill_latent",
    "maba_hip_dgda_layer_prefill_workspace_size",
    "maba_hip_dgda_layer_prefill",
    "maba_hip_dgda_layer_step",
    "maba_hip_decode_linear",
    "maba_hip_argmax_rows",
    "maba_hip_cache_append_heads",
    "maba_hip_maba_sa_decode_dev_heads",
)


class HipLibraryMissing(RuntimeError):
    """The HIP backend library is not built or cannot be loaded."""


class MabaTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * 4),
        ("stride", ctypes.c_int64 * 4),
    ]


_lib = None
_lib_err: Optional[str] = None
_lock = threading.Lock()


def _declare(lib) -> None:
    T = ctypes.POINTER(MabaTensor)
    TA = ctypes.POINTER(T)   # array of descriptor pointers
    vp, i, f, i64, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_int64, ctypes.c_size_t
    sig = {
        "maba_hip_last_error": ([], ctypes.c_char_p),
        "maba_hip_abi_version": ([], i),
        "maba_hip_dgda_prefill_workspace_size": ([T, T, T, T], sz),
        "maba_hip_dgda_prefill": ([T, T, T, T, T, T, T, T, T, T, i, vp, sz, vp], i),
        "maba_hip_dgda_step": ([T, T, T, T, T, T, T, T, T, T, vp], i),
        "maba_hip_compute_centroids": ([T, T, i, vp], i),
        "maba_hip_index_topk": ([T, T, f, i, i, T, T, vp], i),
        "maba_hip_index_topk_decode_workspace_size": ([i64, i64, i64, i], sz),
        "maba_hip_index_topk_decode": ([T, T, f, i, T, T, vp, sz, vp], i),
        "maba_hip_stream_superposition": ([T, T, T, T, i, T, vp], i),
        "maba_hip_hca_pool": ([T, T, i, vp], i),
        "maba_hip_maba_sa_decode_workspace_size": ([i64, i64, i64, i64, i64, i, i, i], sz),
        "maba_hip_maba_sa_decode": ([T, T, T, T, T, i64, f, i, i, i, i, T, vp, sz, vp], i),
        "maba_hip_maba_sa_decode_static": ([T, T, T, T, T, i64, f, i, i, i, i, T, vp], i),
        "maba_hip_dgda_prologue": ([TA, TA, TA, f, TA, TA, vp], i),
        "maba_hip_maba_sa_prefill": ([T, T, T, T, T, T, T, T, f, i, i, i, i, T, vp], i),
        "maba_hip_cache_append": ([T, T, vp, T, T, T, T, i, i, vp], i),
        "maba_hip_index_topk_decode_dev": ([T, T, vp, i, f, i, T, vp, sz, vp], i),
        "maba_hip_maba_sa_decode_dev": ([T, T, T, T, T, vp, i64, f, i, i, i, i, T, vp, sz, vp], i),
        "maba_hip_rmsnorm": ([T, T, T, T, f, T, T, vp], i),
        "maba_hip_swiglu": ([T, T, vp], i),
        "maba_hip_maba_sa_prefill_latent": ([T, T, T, T, T, f, i, i, i, i, T, vp], i),
        "maba_hip_dgda_layer_prefill_workspace_size": ([i64, i64, i64], sz),
        "maba_hip_dgda_layer_prefill": ([TA, TA, TA, f, T, T, T, TA, vp, sz, vp], i),
        "maba_hip_dgda_layer_step": ([TA, TA, TA, f, T, T, T, TA, vp], i),
        "maba_hip_decode_linear": ([T, T, T, T, T, f, i, T, T, T, vp], i),
        "maba_hip_argmax_rows": ([T, T, vp], i),
        "maba_hip_cache_append_heads": ([T, T, vp, T, T, T, T, i, i, T, T, T, T, T, T, vp], i),
        "maba_hip_maba_sa_decode_dev_heads": ([T, T, T, T, T, vp, i64, f, i, i, i, i, T, T, T, vp, sz, vp], i),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res


def load(required: bool = True):
    """Load the library once; raise ``HipLibraryMissing`` when ``required``."""
    global _lib, _lib_err
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None and _lib_err is None:
            if not os.path.exists(LIB_PATH):
                _lib_err = f"{LIB_PATH} not found; run __graft_entry__.build() first"
            else:
                try:
                    lib = ctypes.CDLL(LIB_PATH)
                    _declare(lib)
                    _lib = lib
                except OSError as exc:  # pragma: no cover - depends on the box
                    _lib_err = f"cannot load {LIB_PATH}: {exc}"
    if _lib is None and required:
        raise HipLibraryMissing(_lib_err or "libmaba_hip.so unavailable")
    return _lib


def available() -> bool:
    return load(required=False) is not None


_PAD_SHAPE = ((), (1,), (1, 1), (1, 1, 1), (1, 1, 1, 1))
_PAD_STRIDE = ((), (0,), (0, 0), (0, 0, 0), (0, 0, 0, 0))
_PACK = struct.Struct("<qii4q4q")   # maba_tensor: data, dtype, ndim, shape[4], stride[4]


def _struct(t: torch.Tensor) -> MabaTensor:
    """The ``maba_tensor`` of ``t`` (shape padded with 1, strides with 0, to four dims).  Packed in
    one call and copied into the structure: it runs for every tensor of every op call, and
    per-field ctypes assignments cost three times as much."""
    nd = t.dim()
    if nd > 4:
        raise ValueError(f"descriptor supports at most 4 dims, got {nd}")
    code = _DTYPE_CODES.get(t.dtype)
    if code is None:
        raise TypeError(f"unsupported dtype {t.dtype}")
    return MabaTensor.from_buffer_copy(_PACK.pack(t.data_ptr() if t.numel() > 0 else 0, code, nd, *t.shape,
                                                  *_PAD_SHAPE[4 - nd], *t.stride(), *_PAD_STRIDE[4 - nd]))


def desc(t: Optional[torch.Tensor]):
    """Build a ``maba_tensor`` descriptor (pointer to it) for a tensor, or None."""
    if t is None:
        return None
    return ctypes.byref(_struct(t))


def desc_array(tensors: Sequence[Optional[torch.Tensor]]):
    """A C array of descriptor pointers (``const maba_tensor* const*``); None entries are NULL."""
    T = ctypes.POINTER(MabaTensor)
    return (T * len(tensors))(*[ctypes.pointer(_struct(t)) if t is not None else T() for t in tensors])


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def check(rc: int, what: str) -> None:
    """Map a status code to the Python exception the reference would raise."""
    if rc == MABA_OK:
        return
    msg = (load().maba_hip_last_error() or b"").decode(errors="replace")
    text = f"{what}: {msg}"
    if rc == MABA_ERR_INVALID:
        raise ValueError(text)
    if rc == MABA_ERR_DTYPE:
        raise TypeError(text)
    if rc == MABA_ERR_UNSUPPORTED:
        raise NotImplementedError(text)
    raise RuntimeError(text)


def require_device(tensors: Sequence[Optional[torch.Tensor]], op: str) -> torch.device:
    """All tensors on one ROCm GPU device (the HIP kernels only run there)."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(f"{op}: HIP backend needs GPU tensors, got {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{op}: Expected all tensors to be on the same device, got {dev} and {t.device}")
    if dev is None:
        raise RuntimeError(f"{op}: no tensor given")
    return dev
