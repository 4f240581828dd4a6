"""The part every attention slot of the decoder shares: the fused q / k / v projection and the output
projection (parameters `c_attn`, `c_proj`, as named by the reference's layers so its checkpoints
load, reference src/selective_attention/model.py:41-57), the head split and merge, and a key/value
cache for prefill and decode.

A cache is a dict (the reference's caches are dicts too, model.py:76-93):

    "k", "v"     (B, H, capacity, D) buffers; positions [0, len) are filled
    "len"        the number of cached positions
    "selected"   (B, G, capacity) fp32, selective slots only: the selection each cached key has
                 received from every cached query (G selectors per layer)
"""

from __future__ import annotations

import torch
import torch.nn as nn
from torch import Tensor


class AttentionSlot(nn.Module):
    def __init__(self, config):
        super().__init__()
        width, heads = config.d_model, config.n_heads
        self.n_heads = heads
        self.head_dim = width // heads
        self.d_model = width
        self.dropout = config.dropout
        self.context_length = config.context_length
        self.c_attn = nn.Linear(width, 3 * width, bias=config.bias)
        self.c_proj = nn.Linear(width, width, bias=config.bias)
        self.resid_dropout = nn.Dropout(config.dropout)

    # -- projections ----------------------------------------------------------------------------

    def split(self, qkv: Tensor) -> tuple[Tensor, Tensor, Tensor]:
        """A c_attn output (B, T, 3C), laid out as (B, T, 3, H, D) -> q, k, v as (B, H, T, D) views."""
        parts = qkv.unflatten(-1, (3, self.n_heads, self.head_dim))
        return tuple(parts.select(2, i).transpose(1, 2) for i in range(3))

    def project(self, x: Tensor) -> tuple[Tensor, Tensor, Tensor]:
        """(B, T, C) -> q, k, v (B, H, T, D)."""
        return self.split(self.c_attn(x))

    def emit(self, y: Tensor) -> Tensor:
        """(B, H, T, D) head outputs -> c_proj of the (B, T, C) concatenation."""
        return self.resid_dropout(self.c_proj(y.transpose(1, 2).flatten(2)))

    # -- key / value cache ----------------------------------------------------------------------

    def new_cache(self, batch: int, capacity: int, device, dtype) -> dict:
        """An empty cache of `capacity` positions."""
        shape = (batch, self.n_heads, capacity, self.head_dim)
        return {"k": torch.zeros(shape, device=device, dtype=dtype),
                "v": torch.zeros(shape, device=device, dtype=dtype), "len": 0}

    @staticmethod
    def cache_put(cache: dict, k: Tensor, v: Tensor) -> tuple[int, int]:
        """Writes (B, H, n, D) keys and values at the cache's next n positions; returns the
        position range [start, end) they took."""
        start = cache["len"]
        end = start + k.shape[2]
        if end > cache["k"].shape[2]:
            raise ValueError(f"cache of {cache['k'].shape[2]} positions cannot take positions up to {end}")
        cache["k"][:, :, start:end] = k
        cache["v"][:, :, start:end] = v
        cache["len"] = end
        return start, end

    def prompt_cache(self, k: Tensor, v: Tensor, capacity: int | None) -> dict:
        """A cache holding a prompt's keys and values, with room for `capacity` positions (by default
        the context length, at least the prompt)."""
        b, _, t, _ = k.shape
        cache = self.new_cache(b, max(t, self.context_length if capacity is None else capacity), k.device, k.dtype)
        self.cache_put(cache, k, v)
        return cache
