"""DG-Indexer layer: caller of ``compute_centroids``, ``index_topk`` and the decode
scoring (reference: layers/indexer.py:9-126).

Semantics follow the reference branch for branch (indexer.py:43-126):

* ``past_k_idx`` given: centroids of the whole key sequence;
* eval decode with a cache: the new key joins the cache; a completed block adds
  one centroid, otherwise the zero-padded tail block's centroid is appended for
  this step only (indexer.py:62-81);
* ``past_centroids`` given: the new tokens' centroids are appended;
* otherwise the centroids of ``x``'s keys, cached when prefilling in eval mode.

A single decode token (``l == 1`` with history, or more than one block) scores
``(q/sqrt d).c_n - lam*log1p(max(nb-1-n, 0))`` and keeps the top ``min(k, nb)``
(indexer.py:101-112) through the ``index_topk_decode`` op; everything else goes
through ``index_topk``.

The key cache is a capacity-doubling buffer rather than a ``torch.cat`` per
step, so a decode step costs O(block) instead of O(L); the centroid cache grows
the same way.  Results are those of the reference's concatenations.
"""
from __future__ import annotations

import math
from typing import Any, Optional, Tuple

import torch
import torch.nn as nn

from maba_sparse.kernels.dispatcher import (dispatch_compute_centroids, dispatch_index_topk,
                                            dispatch_index_topk_decode)


class _Growing:
    """Rows ``[B, n, d]`` appended along dim 1 into a buffer that doubles when full."""

    def __init__(self, init: torch.Tensor):
        cap = max(64, 1 << max(0, int(init.shape[1]) - 1).bit_length())
        self.buf = init.new_empty(init.shape[0], cap, init.shape[2])
        self.n = int(init.shape[1])
        self.buf[:, : self.n] = init

    def append(self, rows: torch.Tensor) -> None:
        m = int(rows.shape[1])
        if self.n + m > self.buf.shape[1]:
            cap = self.buf.shape[1]
            while cap < self.n + m:
                cap *= 2
            nb = self.buf.new_empty(self.buf.shape[0], cap, self.buf.shape[2])
            nb[:, : self.n] = self.buf[:, : self.n]
            self.buf = nb
        self.buf[:, self.n: self.n + m] = rows
        self.n += m

    def view(self) -> torch.Tensor:
        return self.buf[:, : self.n]

    def view_with(self, row: torch.Tensor) -> torch.Tensor:
        """The rows plus ``row [B, 1, d]`` in the next slot, without appending it: the
        next ``append`` overwrites the slot.  No copy of the held rows."""
        self.append(row)
        self.n -= 1
        return self.buf[:, : self.n + 1]

    @property
    def shape(self) -> torch.Size:
        return torch.Size([self.buf.shape[0], self.n, self.buf.shape[2]])


class DGIndexer(nn.Module):
    def __init__(self, dim: int = 640, d_idx: int = 64, block_size: int = 64, top_k: int = 32,
                 dist_lambda: float = 0.5, config: Optional[Any] = None) -> None:
        super().__init__()
        if config is not None:
            dim = getattr(config, "dim", getattr(config, "d_model", dim))
            d_idx = getattr(config, "d_idx", d_idx)
            block_size = getattr(config, "block_size", block_size)
            top_k = getattr(config, "top_k", top_k)
            dist_lambda = getattr(config, "dist_lambda", dist_lambda)
        self.dim, self.d_idx, self.block_size = dim, d_idx, block_size
        self.top_k, self.dist_lambda = top_k, dist_lambda
        self.q_idx_proj = nn.Linear(dim, d_idx, bias=False)
        self.k_idx_proj = nn.Linear(dim, d_idx, bias=False)
        self.scale = 1.0 / math.sqrt(d_idx)
        self._keys: Optional[_Growing] = None       # cached k_idx rows (eval decode)
        self._cents: Optional[_Growing] = None      # centroids of the complete cached blocks

    # reference attribute names (indexer.py:36-37), as read-only views
    @property
    def _cached_k_idx(self) -> Optional[torch.Tensor]:
        return None if self._keys is None else self._keys.view()

    @property
    def _cached_centroids(self) -> Optional[torch.Tensor]:
        return None if self._cents is None or self._cents.n == 0 else self._cents.view()

    def reset_cache(self) -> None:
        self._keys = None
        self._cents = None

    def restore_cache(self, k_idx: torch.Tensor) -> None:
        """Set the decode cache to the key rows ``k_idx [B, L, d_idx]`` of a held sequence, as a
        prefill of those tokens leaves it: the rows, and the centroids of their complete blocks."""
        self._keys = _Growing(k_idx.detach())
        full = k_idx.shape[1] // self.block_size
        self._cents = (_Growing(dispatch_compute_centroids(k_idx[:, : full * self.block_size].detach(),
                                                           block_size=self.block_size)) if full > 0 else None)

    def _centroids(self, ki: torch.Tensor, past_centroids, past_k_idx) -> torch.Tensor:
        b, l, _ = ki.shape
        bs = self.block_size
        if past_k_idx is not None:
            return dispatch_compute_centroids(torch.cat([past_k_idx, ki], dim=1), block_size=bs)
        if not self.training and l == 1 and self._keys is not None and self._keys.shape[0] == b:
            self._keys.append(ki.detach())
            n = self._keys.n
            rem = n % bs
            if rem == 0:
                new_c = dispatch_compute_centroids(self._keys.view()[:, n - bs:], block_size=bs)
                if self._cents is None:
                    self._cents = _Growing(new_c)
                else:
                    self._cents.append(new_c)
                return self._cents.view()
            tail = dispatch_compute_centroids(self._keys.view()[:, n - rem:], block_size=bs)
            if self._cents is None or self._cents.n == 0:
                return tail
            # the zero-padded tail centroid joins the complete ones for this step only
            # (indexer.py:75-81), written into the cache's next slot instead of a concatenation
            return self._cents.view_with(tail)
        if past_centroids is not None:
            return torch.cat([past_centroids, dispatch_compute_centroids(ki, block_size=bs)], dim=1)
        c = dispatch_compute_centroids(ki, block_size=bs)
        if not self.training and l > 1:
            self._keys = _Growing(ki.detach())
            full = l // bs
            self._cents = _Growing(c[:, :full].detach()) if full > 0 else None
        else:
            self.reset_cache()
        return c

    def forward(self, x: torch.Tensor, top_k: Optional[int] = None, dist_lambda: Optional[float] = None,
                return_scores: bool = False, past_centroids: Optional[torch.Tensor] = None,
                past_k_idx: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, ...]:
        return self.forward_projected(self.q_idx_proj(x), self.k_idx_proj(x), top_k, dist_lambda, return_scores,
                                      past_centroids, past_k_idx)

    def forward_projected(self, qi: torch.Tensor, ki: torch.Tensor, top_k: Optional[int] = None,
                          dist_lambda: Optional[float] = None, return_scores: bool = False,
                          past_centroids: Optional[torch.Tensor] = None,
                          past_k_idx: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, ...]:
        """``forward`` from the query and key projections ``q_idx_proj(x)``, ``k_idx_proj(x)``
        (a caller that projects the token once for several modules passes them in)."""
        b, l, _ = qi.shape
        k = self.top_k if top_k is None else top_k
        lam = self.dist_lambda if dist_lambda is None else dist_lambda
        c = self._centroids(ki, past_centroids, past_k_idx)
        nb = c.shape[1]
        if l == 1 and (past_centroids is not None or past_k_idx is not None or nb > 1):
            res = dispatch_index_topk_decode(qi, c, lambda_dist=lam, top_k=k, return_scores=return_scores)
            if return_scores:
                idx, sc = res
                return idx, c, sc.to(qi.dtype)
            return res, c
        res = dispatch_index_topk(q_idx=qi, centroids=c, lambda_dist=lam, top_k=k,
                                  block_size=self.block_size, return_scores=return_scores)
        if return_scores:
            idx, sc = res
            return idx, c, sc
        return res, c


DeltaGuidedCentroidIndexer = DGIndexer
