"""Selective Attention as an attention slot of a decoder (reference src/selective_attention/mixers.py).

`VARIANTS` / `MIXER_TYPES` / `MIXER_CLASSES` keep the reference's names (mixers.py:21-32), so a
model config selects the layer with `attention: selective | selective_x16 | selective_perhead`:

    selective           head 0 selects for every head, <BOS> (position 0) exempt
    selective_x16       the first 16 positions are exempt
    selective_perhead   every head selects for itself (each head runs as a one-head sequence)

The layer routes every call through the HIP kernels (kernels.py). There is no silent fallback: a
layer whose inputs the kernels cannot take raises, and the plain (T x T) listing runs only when the
caller asks for it with `use_kernel = False` (CPU runs, debugging).

Cached generation keeps, per sequence and selector, the selection every key has received so far
(reference mixers.py:105-130): a prefill (single shot, or chunk by chunk with `prefill_chunk`)
leaves it in the cache, and each decode step subtracts it from every head's logits and then adds
the new query's own relu'd selector logits.
"""

from __future__ import annotations

import math

import torch
from torch import Tensor

from . import kernels

# name: (exempt, per_head)
VARIANTS = {"selective": (1, False), "selective_x16": (16, False), "selective_perhead": (1, True)}
MIXER_TYPES = tuple(VARIANTS)


def __getattr__(name: str):
    # built on first use: the layer class needs model._AttentionBase, and model imports this module
    if name == "MIXER_CLASSES":
        cls = selective_class()
        return {kind: (lambda config, e=e, p=p: cls(config, exempt=e, per_head=p))
                for kind, (e, p) in VARIANTS.items()}
    raise AttributeError(name)


_CLASS = None


def selective_class():
    """The SelectiveAttention layer class (defined lazily, see __getattr__)."""

    global _CLASS
    if _CLASS is None:
        from .model import _AttentionBase

        class SelectiveAttention(_AttentionBase):
            """softmax(L - F) attention with the q / k / v / output projections every attention
            layer has and no other parameters (reference mixers.py:50-130)."""

            def __init__(self, config, exempt: int = 1, per_head: bool = False):
                super().__init__(config)
                self.exempt = kernels._check_exempt(exempt)
                self.groups = self.n_heads if per_head else 1   # selectors per layer
                self.use_kernel = True
                self.history_damp = "none"   # evaluation-only history scaling of the forward
                self.dot_precision = None    # None: bf16 operands for bf16 inputs, else fp32

            # -- routing -----------------------------------------------------------------------

            def _check_kernel(self, q: Tensor) -> None:
                if self.training and self.dropout > 0.0:
                    raise RuntimeError("selective attention kernels have no attention dropout; set dropout=0")
                kernels.check_inputs(q, q, q)   # raises with the reason (device, dtype, head_dim, library)

            def _grouped(self, *ts: Tensor) -> tuple[Tensor, ...]:
                """(B, H, T, D) -> (B*G, H/G, T, D): each group of heads is its own sequence, so its
                first head selects (reference mixers.py:76-84)."""
                b, h, t, d = ts[0].shape
                return tuple(x.reshape(b * self.groups, h // self.groups, x.shape[2], d) for x in ts)

            def _attend(self, q: Tensor, k: Tensor, v: Tensor, want_total: bool = False):
                """(B, H, T, D) outputs in v's dtype and, on request, the (B, G, T) selection totals."""
                b, h, t, d = q.shape
                qg, kg, vg = self._grouped(q, k, v)
                if not self.use_kernel:
                    with torch.autocast(q.device.type, enabled=False):
                        logits, total = kernels.selective_logits(qg, kg, self.exempt)
                        y = (logits.softmax(dim=-1) @ vg.float()).to(v.dtype)
                else:
                    self._check_kernel(qg)
                    if want_total or not torch.is_grad_enabled():
                        y, aux = kernels.selective_attention_forward(
                            qg, kg, vg, dot_precision=self.dot_precision, return_aux=True, exempt=self.exempt,
                            damp=self.history_damp, train_len=self.context_length)
                        y, total = y.to(v.dtype), aux["selected_total"]
                    else:
                        y = kernels.selective_attention(qg, kg, vg, dot_precision=self.dot_precision,
                                                        exempt=self.exempt).to(v.dtype)
                        total = None
                y = y.reshape(b, h, t, d)
                return y, (None if total is None else total.reshape(b, self.groups, t))

            def forward(self, x: Tensor) -> Tensor:
                b, t, _ = x.shape
                qkv = self.c_attn(x)
                if (self.use_kernel and self.groups == 1 and self.history_damp in (None, "none")
                        and kernels.packed_supported(qkv, self.n_heads, self.dot_precision)):
                    # layer-boundary fused form: q, k, v read in place from the projection, the
                    # output written in the layout c_proj reads, the gradient as one tensor
                    if self.training and self.dropout > 0.0:
                        raise RuntimeError("selective attention kernels have no attention dropout; set dropout=0")
                    y = kernels.selective_attention_qkv(qkv, self.n_heads, self.dot_precision, self.exempt)
                    return self.resid_dropout(self.c_proj(y))
                hd = self.d_model // self.n_heads
                qkv = qkv.view(b, t, 3, self.n_heads, hd)
                q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
                return self._merge_heads(self._attend(q, k, v)[0], b, t)

            # -- cached generation ---------------------------------------------------------------

            def begin_cache(self, x: Tensor, capacity: int | None = None):
                """Single-shot prefill: outputs and a cache of K, V and the per-key selection."""
                b, t, _ = x.shape
                q, k, v = self._split_heads(x)
                y, total = self._attend(q, k, v, want_total=True)
                cache = self._alloc_cache(k, v, capacity)
                cache["selected"] = torch.zeros(b, self.groups, cache["k"].shape[2], device=x.device,
                                                dtype=torch.float32)
                cache["selected"][:, :, :t] = total.float()
                return self._merge_heads(y, b, t), cache

            def new_cache(self, batch: int, capacity: int, device, dtype) -> dict:
                """An empty cache for `prefill_chunk` (K, V in `dtype`, selection state fp32)."""
                hd = self.d_model // self.n_heads
                return {"k": torch.zeros(batch, self.n_heads, capacity, hd, device=device, dtype=dtype),
                        "v": torch.zeros(batch, self.n_heads, capacity, hd, device=device, dtype=dtype),
                        "selected": torch.zeros(batch, self.groups, capacity, device=device, dtype=torch.float32),
                        "len": 0}

            def prefill_chunk(self, x: Tensor, cache: dict) -> Tensor:
                """The next chunk of a chunked prefill: appends its K, V to the cache and attends
                with the selection state carried from the earlier chunks (no reference counterpart:
                the reference runs long inputs as one forward, kernels.py:38-40)."""
                if not self.use_kernel:
                    raise RuntimeError("prefill_chunk runs the HIP kernels; use begin_cache with use_kernel=False")
                b, tc, _ = x.shape
                c0 = cache["len"]
                c1 = c0 + tc
                if c1 > cache["k"].shape[2]:
                    raise ValueError("prefill chunk past the cache capacity")
                q, k, v = self._split_heads(x, offset=c0)
                cache["k"][:, :, c0:c1] = k
                cache["v"][:, :, c0:c1] = v
                cache["len"] = c1
                self._check_kernel(q)
                keys, vals = cache["k"][:, :, :c1], cache["v"][:, :, :c1]
                state = cache["selected"].view(b * self.groups, -1)
                if self.groups == 1:
                    y = kernels.selective_attention_prefill(q, keys, vals, state, c0, dot_precision=self.dot_precision,
                                                            exempt=self.exempt)
                else:
                    qg, kg, vg = self._grouped(q, keys, vals)
                    y = kernels.selective_attention_prefill(qg, kg, vg, state, c0, dot_precision=self.dot_precision,
                                                            exempt=self.exempt)
                return self._merge_heads(y.reshape(b, self.n_heads, tc, -1).to(v.dtype), b, tc)

            def step_cache(self, x1: Tensor, cache: dict) -> Tensor:
                """One decode step (reference mixers.py:115-130): subtract the carried selection from
                every head's logits, then add this query's own selection to the state. With
                use_kernel, one HIP launch pair (kernels.selective_attention_decode); otherwise the
                reference's PyTorch step."""
                b = x1.shape[0]
                q1, k1, v1 = self._split_heads(x1, offset=cache["len"])
                t = self._append_kv(cache, k1, v1)
                keys, vals = cache["k"][:, :, :t], cache["v"][:, :, :t]
                if self.use_kernel:
                    self._check_kernel(q1)
                    y = kernels.selective_attention_decode(q1, keys, vals, cache["selected"], exempt=self.exempt)
                    return self._merge_heads(y[:, :, None].to(x1.dtype), b, 1)
                selected = cache["selected"][:, :, :t]                   # (B, G, t)
                per = self.n_heads // self.groups
                with torch.autocast(x1.device.type, enabled=False):
                    raw = (q1.float() @ keys.float().transpose(-2, -1)) / math.sqrt(self.d_model // self.n_heads)
                    hist = selected.repeat_interleave(per, dim=1)[:, :, None, :]
                    y = ((raw - hist).softmax(dim=-1) @ vals.float()).to(x1.dtype)
                    own = torch.relu(raw[:, ::per, 0])               # the selector head of each group
                    own[..., : self.exempt] = 0.0                    # exempt positions are never selected
                    own[..., t - 1] = 0.0                            # nor is the query's own key
                    selected += own
                return self._merge_heads(y, b, 1)

        SelectiveAttention.__module__ = __name__
        _CLASS = SelectiveAttention
    return _CLASS
