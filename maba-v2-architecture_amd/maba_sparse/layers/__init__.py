"""Callers of the hot-path ops, mirroring maba_sparse/layers in the reference."""
from maba_sparse.layers.dgda import ConvState, DecoupledGatedDeltaAttention, DGDALayer
from maba_sparse.layers.indexer import DeltaGuidedCentroidIndexer, DGIndexer
from maba_sparse.layers.sparse_attention import LatentCache, MABASALayer, MabaSparseAttention

__all__ = ["ConvState", "DGDALayer", "DecoupledGatedDeltaAttention", "DGIndexer", "DeltaGuidedCentroidIndexer",
           "LatentCache", "MabaSparseAttention", "MABASALayer"]
