"""On-disk format of a model's decode state: everything ``step`` reads after a prefill.

The reference keeps its decode state in memory only (``forward``/``step`` pass
``past_states``, model.py:207-270; ``train.py:249-261`` saves weights only).  This module
writes that state to one safetensors file and reads it back, so a served sequence can be
paused, moved to another process or device, and resumed with ``step`` (or the HIP
serving loop) giving the same logits as an uninterrupted run.

A resumed MABA-SA block also needs its indexer's key cache: the reference's layer drops it
when ``past_c_kv`` arrives without it (layers/sparse_attention.py:228-233 resets the caches
whose length differs), after which the decode indexer scores only the new token's block.
The file therefore carries the indexer key rows, and ``load_decode_state`` restores them.

Format (version 1).  Metadata (strings): ``format = "maba-decode-state"``, ``version = "1"``,
``n_layers``, ``length`` (tokens held), ``kinds`` (one letter per layer: ``d`` DGDA, ``a``
MABA-SA).  Tensors, in the dtypes they had in memory:

- ``layers.{i}.state``: DGDA recurrent state ``[B, H, d_k, d_v]``;
- ``layers.{i}.conv_q``, ``.conv_k``, ``.conv_v``: DGDA conv histories ``[B, C, kernel - 1]``;
- ``layers.{i}.c_kv``: MABA-SA latent rows ``[B, L, d_c]``;
- ``layers.{i}.k_idx``: that block's indexer key rows ``[B, L, d_idx]``.
"""
from __future__ import annotations

from typing import Any, List, Optional

import torch

FORMAT = "maba-decode-state"
VERSION = "1"


def save_decode_state(model, past_states: List[Any], path: str) -> None:
    """Write ``past_states`` (the list ``forward``/``step`` return, one ``(state, conv_state,
    c_kv)`` per block) and the MABA-SA blocks' indexer key caches to ``path``."""
    from safetensors.torch import save_file
    layers = model.layers
    if len(past_states) != len(layers):
        raise ValueError(f"save_decode_state: {len(past_states)} layer states for {len(layers)} layers")
    tensors, kinds, length = {}, [], None
    for i, (layer, (st, cv, ck)) in enumerate(zip(layers, past_states)):
        if layer.is_attention:
            keys = layer.mixer.indexer._cached_k_idx
            if ck is None or keys is None or keys.shape[1] != ck.shape[1]:
                raise ValueError(f"save_decode_state: layer {i} holds no latent rows with a matching indexer cache "
                                 "(run a prefill in eval mode first)")
            tensors[f"layers.{i}.c_kv"] = ck
            tensors[f"layers.{i}.k_idx"] = keys
            if length is not None and ck.shape[1] != length:
                raise ValueError("save_decode_state: MABA-SA blocks hold different lengths")
            length = ck.shape[1]
            kinds.append("a")
        else:
            if st is None or cv is None:
                raise ValueError(f"save_decode_state: layer {i} has no DGDA state")
            tensors[f"layers.{i}.state"] = st
            for name, h in zip(("conv_q", "conv_k", "conv_v"), cv):
                tensors[f"layers.{i}.{name}"] = h
            kinds.append("d")
    meta = {"format": FORMAT, "version": VERSION, "n_layers": str(len(layers)), "length": str(length or 0),
            "kinds": "".join(kinds)}
    save_file({k: v.detach().contiguous() for k, v in tensors.items()}, path, metadata=meta)


def load_decode_state(model, path: str, device: Optional[torch.device] = None) -> List[Any]:
    """Read a file written by ``save_decode_state`` for a model of the same architecture:
    returns ``past_states`` for ``step`` and restores the MABA-SA blocks' indexer caches."""
    from safetensors import safe_open
    from maba_sparse.layers.dgda import ConvState
    dev = device if device is not None else next(model.parameters()).device
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT:
            raise ValueError(f"load_decode_state: {path} is not a {FORMAT} file")
        if meta.get("version") != VERSION:
            raise ValueError(f"load_decode_state: unsupported version {meta.get('version')!r} (this reads {VERSION})")
        kinds = meta.get("kinds", "")
        if len(kinds) != len(model.layers) or any((k == "a") != l.is_attention for k, l in zip(kinds, model.layers)):
            raise ValueError(f"load_decode_state: the file's block pattern {kinds!r} does not match the model")
        states: List[Any] = []
        for i, layer in enumerate(model.layers):
            if layer.is_attention:
                ck = f.get_tensor(f"layers.{i}.c_kv").to(dev)
                keys = f.get_tensor(f"layers.{i}.k_idx").to(dev)
                layer.mixer.reset_cache()
                layer.mixer.indexer.restore_cache(keys)
                states.append((None, None, ck))
            else:
                st = f.get_tensor(f"layers.{i}.state").to(dev)
                cv = ConvState(tuple(f.get_tensor(f"layers.{i}.{n}").to(dev) for n in ("conv_q", "conv_k", "conv_v")))
                states.append((st, cv, None))
    return states
