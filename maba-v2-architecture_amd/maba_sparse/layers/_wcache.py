"""Weight-derived tensors kept between inference calls, and their invalidation.

The decode paths stack several projection weights into one GEMM operand, convert
head views to fp32 or cache gate sigmoids, so that a serving step does not rebuild
them per token.  Each such tensor is stored on its module under a ``_wcache_`` key
with a tag of the source parameters' ``(data_ptr, _version, dtype, device)``: an
in-place update through the parameter (``p.copy_``, ``p.mul_``, ``load_state_dict``)
bumps ``_version`` and a move (``.to``) changes the pointer, so both rebuild the
tensor on the next call.

A write through ``p.data`` (``p.data.copy_(...)``) bumps no version counter and
cannot be seen from the tag.  After such a write call ``clear_weight_caches()`` on
the module (or any parent); ``MabaSparseForCausalLM.generate_greedy`` calls it on
entry, and ``load_state_dict`` and ``_apply`` (``.to``, ``.cuda``, ``.half``) call
it as well.
"""
from __future__ import annotations

from typing import Callable, Sequence

import torch
import torch.nn as nn

PREFIX = "_wcache_"


def cached(module: nn.Module, key: str, params: Sequence[torch.Tensor], build: Callable[[], torch.Tensor]):
    """``build()``, kept on ``module`` until one of ``params`` changes.  Under autograd with a
    parameter that requires grad the value is rebuilt every call (it must carry the graph)."""
    if torch.is_grad_enabled() and any(p.requires_grad for p in params):
        return build()
    tag = tuple((p.data_ptr(), p._version, p.dtype, p.device) for p in params)
    held = module.__dict__.get(PREFIX + key)
    if held is None or held[0] != tag:
        held = (tag, build())
        module.__dict__[PREFIX + key] = held
    return held[1]


def clear_weight_caches(module: nn.Module) -> None:
    """Drop every weight-derived tensor held by ``module`` and its submodules."""
    for m in module.modules():
        for k in [k for k in m.__dict__ if k.startswith(PREFIX)]:
            del m.__dict__[k]


class WeightCacheMixin:
    """``clear_weight_caches()`` for an ``nn.Module``, also run after ``load_state_dict`` and
    after ``_apply`` (device and dtype moves)."""

    def clear_weight_caches(self) -> None:
        clear_weight_caches(self)

    def _install_weight_cache_hooks(self) -> None:
        self.register_load_state_dict_post_hook(lambda mod, incompatible: clear_weight_caches(mod))

    def _apply(self, fn, *args, **kwargs):
        out = super()._apply(fn, *args, **kwargs)
        clear_weight_caches(self)
        return out

    def __getstate__(self):
        # copies and pickles start without caches: a cached tensor may be a view of a
        # parameter (fp32 weights convert to themselves), which deepcopy cannot always copy
        state = super().__getstate__()
        return {k: v for k, v in state.items() if not k.startswith(PREFIX)}
