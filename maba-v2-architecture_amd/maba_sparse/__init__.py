"""Maba v2 hot path on MI355X (gfx950): dispatcher-compatible kernel ops backed by
hand-written HIP kernels, plus the layer-level callers of those ops.

``maba_sparse.kernels`` mirrors the reference package's kernel API
(``maba_sparse/kernels/__init__.py`` of the reference) with a ``"hip"`` backend;
``maba_sparse.layers`` holds the DGDA, DG-Indexer and MABA-SA callers.
"""
__version__ = "0.1.0"
