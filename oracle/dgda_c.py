"""ctypes binding of ``oracle/dgda_chunked.c`` -- TEST INFRASTRUCTURE ONLY.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg.  ``build()`` runs ``make -C oracle``; the shared library
lands in ``oracle/_build/``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle_dgda.so")
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        fp = ctypes.POINTER(ctypes.c_float)
        i = ctypes.c_int
        lib.oracle_dgda_prefill_f32.argtypes = [i, i, i, i, i, i, fp, fp, fp, fp, i, fp, i, fp, i,
                                                fp, fp, fp, i]
        lib.oracle_dgda_prefill_f32.restype = i
        lib.oracle_max_threads.restype = i
        _lib = lib
    return _lib


def max_threads() -> int:
    return _load().oracle_max_threads()


def _gate(g, shape_full):
    """Return (contiguous float32 array, per_channel flag) for a gate.

    A gate whose last axis has size 1 (or is constant along the channel axis by
    construction, passed as ``[B,H,L]``) is handed over per token.
    """
    g = np.asarray(g, np.float32)
    if g.ndim == 3:
        return np.ascontiguousarray(g), 0
    if g.shape[-1] == 1:
        return np.ascontiguousarray(g[..., 0]), 0
    assert g.shape == shape_full, (g.shape, shape_full)
    return np.ascontiguousarray(g), 1


def dgda_prefill_chunked_c(q, k, v, log_alpha, b, w, initial_state=None, chunk_size=64,
                           nthreads=0):
    """Chunked fp32 DGDA prefill (cpu_dgda.py:33-197).  Gates may be per token
    (``[B,H,L]`` / trailing size-1 axis) or per channel."""
    lib = _load()
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    B, H, L, dk = q.shape
    dv = v.shape[-1]
    la, la_pc = _gate(log_alpha, (B, H, L, dk))
    bg, b_pc = _gate(b, (B, H, L, dk))
    wg, w_pc = _gate(w, (B, H, L, dv))
    s0 = None if initial_state is None else np.ascontiguousarray(initial_state, np.float32)
    out = np.empty((B, H, L, dv), np.float32)
    sf = np.empty((B, H, dk, dv), np.float32)
    P = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    rc = lib.oracle_dgda_prefill_f32(B, H, L, dk, dv, chunk_size, P(q), P(k), P(v), P(la), la_pc,
                                     P(bg), b_pc, P(wg), w_pc,
                                     None if s0 is None else P(s0), P(out), P(sf), int(nthreads))
    if rc != 0:
        raise RuntimeError(f"oracle_dgda_prefill_f32 failed with code {rc}")
    return out, sf
