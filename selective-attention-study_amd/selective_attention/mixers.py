"""Selective Attention as an attention slot of a decoder (reference src/selective_attention/mixers.py).

`VARIANTS` / `MIXER_TYPES` / `MIXER_CLASSES` keep the reference's names (mixers.py:21-32), so a
model config selects the layer with `attention: selective | selective_x16 | selective_perhead`:

    selective           head 0 selects for every head, <BOS> (position 0) exempt
    selective_x16       the first 16 positions are exempt
    selective_perhead   every head selects for itself (each head runs as a one-head sequence)

Routing (reference mixers.py:73-74, 87-98): calls on CUDA (ROCm) tensors run the HIP kernels of
`kernels`; CPU tensors, `use_kernel = False`, a head dim the kernels do not take, or attention
dropout in training run the plain (T x T) listing, `kernels.selective_logits`, as the reference
does. On a GPU tensor whose shape the kernels take, a missing HIP library is an error, never a
silent switch to the listing.

Cached generation keeps, per sequence and selector, the selection every key has received so far: a
prefill (single shot, or chunk by chunk with `prefill_chunk`) leaves it in the cache, and each
decode step subtracts it from every head's logits and then adds the new query's own positive
selector logits (keys past the exempt prefix, before the query).
"""

from __future__ import annotations

import functools
import math

import torch
from torch import Tensor

from . import _lib, kernels
from .slot import AttentionSlot

# name: (exempt, per_head)
VARIANTS = {"selective": (1, False), "selective_x16": (16, False), "selective_perhead": (1, True)}
MIXER_TYPES = tuple(VARIANTS)


class SelectiveAttention(AttentionSlot):
    """softmax(L - F) attention with the q / k / v / output projections every attention layer has
    and no other parameters (reference mixers.py:50-130)."""

    def __init__(self, config, exempt: int = 1, per_head: bool = False):
        super().__init__(config)
        self.exempt = kernels._check_exempt(exempt)
        self.groups = self.n_heads if per_head else 1   # selectors per layer
        self.use_kernel = True
        self.history_damp = "none"   # evaluation-only history scaling of the kernel forward
        self.dot_precision = None    # None: bf16 operands for bf16 inputs, else fp32

    # -- routing ----------------------------------------------------------------------------------

    def _on_kernels(self, x: Tensor) -> bool:
        """Whether a call on x (a q, or the projection it comes from) runs the HIP kernels."""
        if not (self.use_kernel and x.is_cuda):
            return False
        if self.training and self.dropout > 0.0:
            return False   # the kernels have no attention dropout
        if not kernels.HAS_HIP:
            _lib.load()    # a GPU box without the library: raise with the reason
        return self.head_dim in kernels.HEAD_DIMS and x.dtype in kernels.DTYPES

    def _sequences(self, x: Tensor) -> Tensor:
        """(B, H, T, D) -> (B*G, H/G, T, D): every head group is its own sequence, whose first head
        selects for it."""
        b, h = x.shape[:2]
        return x.reshape(b * self.groups, h // self.groups, *x.shape[2:])

    def _listing(self, q: Tensor, k: Tensor, v: Tensor) -> tuple[Tensor, Tensor]:
        """The (T x T) listing on (sequences, heads, T, D): fp32 outputs and the per-key totals."""
        with torch.autocast(q.device.type, enabled=False):
            z, total = kernels.selective_logits(q, k, self.exempt)
            return torch.softmax(z, dim=-1) @ v.float(), total

    def _attend(self, q: Tensor, k: Tensor, v: Tensor, want_total: bool = False):
        """(B, H, T, D) outputs in v's dtype and, on request, the (B, G, T) selection totals."""
        b, h, t, d = q.shape
        qs, ks, vs = (self._sequences(x) for x in (q, k, v))
        total = None
        if not self._on_kernels(q):
            y, total = self._listing(qs, ks, vs)
        elif want_total or not torch.is_grad_enabled():
            y, aux = kernels.selective_attention_forward(
                qs, ks, vs, dot_precision=self.dot_precision, return_aux=True, exempt=self.exempt,
                damp=self.history_damp, train_len=self.context_length)
            total = aux["selected_total"]
        else:
            y = kernels.selective_attention(qs, ks, vs, dot_precision=self.dot_precision, exempt=self.exempt)
        y = y.to(v.dtype).reshape(b, h, t, d)
        return y, (None if total is None or not want_total else total.reshape(b, self.groups, t))

    def forward(self, x: Tensor) -> Tensor:
        qkv = self.c_attn(x)
        if (self.groups == 1 and self.history_damp in (None, "none") and self._on_kernels(qkv)
                and kernels.packed_supported(qkv, self.n_heads, self.dot_precision)):
            # layer-boundary fused form: q, k, v read in place from the projection, the output
            # written in the layout c_proj reads, the gradient as one tensor
            return self.resid_dropout(self.c_proj(
                kernels.selective_attention_qkv(qkv, self.n_heads, self.dot_precision, self.exempt)))
        q, k, v = self.split(qkv)
        return self.emit(self._attend(q, k, v)[0])

    # -- cached generation ----------------------------------------------------------------------

    def new_cache(self, batch: int, capacity: int, device, dtype) -> dict:
        """An empty cache for `prefill_chunk`: K, V in `dtype`, the selection state in fp32."""
        cache = super().new_cache(batch, capacity, device, dtype)
        cache["selected"] = torch.zeros(batch, self.groups, capacity, device=device, dtype=torch.float32)
        return cache

    def begin_cache(self, x: Tensor, capacity: int | None = None):
        """Single-shot prefill: the outputs and a cache of K, V and the per-key selection."""
        q, k, v = self.project(x)
        y, total = self._attend(q, k, v, want_total=True)
        cache = self.prompt_cache(k, v, capacity)
        cache["selected"][:, :, :k.shape[2]] = total
        return self.emit(y), cache

    def prefill_chunk(self, x: Tensor, cache: dict) -> Tensor:
        """The next chunk of a chunked prefill: appends its K, V to the cache and attends with the
        selection state carried from the earlier chunks (no reference counterpart: the reference
        runs long inputs as one forward, kernels.py:38-40)."""
        q, k, v = self.project(x)
        c0, c1 = self.cache_put(cache, k, v)
        keys, vals = cache["k"][:, :, :c1], cache["v"][:, :, :c1]
        state = cache["selected"]
        if self._on_kernels(q):
            b = q.shape[0]
            y = kernels.selective_attention_prefill(self._sequences(q), self._sequences(keys), self._sequences(vals),
                                                    state.view(b * self.groups, -1), c0,
                                                    dot_precision=self.dot_precision, exempt=self.exempt)
            y = y.reshape(q.shape)
        else:
            y = self._chunk_listing(q, keys, vals, state, c0)
        return self.emit(y.to(v.dtype))

    def step_cache(self, x1: Tensor, cache: dict) -> Tensor:
        """One decode step (reference mixers.py:115-130): subtract the carried selection from every
        head's logits, then add this query's own selection to the state. On the kernels, one HIP
        launch pair (kernels.selective_attention_decode)."""
        q1, k1, v1 = self.project(x1)
        _, t = self.cache_put(cache, k1, v1)
        keys, vals = cache["k"][:, :, :t], cache["v"][:, :, :t]
        if self._on_kernels(q1):
            y = kernels.selective_attention_decode(q1, keys, vals, cache["selected"], exempt=self.exempt)[:, :, None]
        else:
            y = self._chunk_listing(q1, keys, vals, cache["selected"], t - 1)
        return self.emit(y.to(x1.dtype))

    def _chunk_listing(self, q: Tensor, keys: Tensor, vals: Tensor, state: Tensor, c0: int) -> Tensor:
        """Queries at positions [c0, c0 + n) over the cached keys [0, c0 + n) with the carried
        per-key selection state (B, G, >= c0 + n) fp32, written out from the operator's definition:
        F[i, j] = state[j] + the selection of key j by this chunk's queries before i. The state is
        advanced by the chunk's selection (in place). A decode step is the chunk of one query."""
        b, h, n, d = q.shape
        g, t = self.groups, c0 + n
        with torch.autocast(q.device.type, enabled=False):
            scores = (q.float() @ keys.float().transpose(-2, -1)) / math.sqrt(d)      # (B, H, n, t)
            grouped = scores.reshape(b, g, h // g, n, t)
            pos = torch.arange(t, device=q.device)
            rows = pos[c0:t, None]                                                   # absolute query positions
            sel = torch.where((pos >= self.exempt) & (pos < rows), grouped[:, :, 0].clamp_min(0.0),
                              torch.zeros((), device=q.device))                       # (B, G, n, t)
            before = torch.cumsum(sel, dim=2) - sel                                   # this chunk's earlier rows
            hist = state[:, :, None, :t] + before                                     # (B, G, n, t)
            z = (grouped - hist[:, :, None]).masked_fill(pos > rows, float("-inf"))
            y = torch.softmax(z, dim=-1) @ vals.float().reshape(b, g, h // g, t, d)
            state[:, :, :t] += sel.sum(dim=2)
        return y.reshape(b, h, n, d)


# name -> factory(config), the registry the decoder's slot table is extended with (reference
# mixers.py:25-32, model.py:306-314)
MIXER_CLASSES = {name: functools.partial(SelectiveAttention, exempt=e, per_head=p) for name, (e, p) in VARIANTS.items()}
