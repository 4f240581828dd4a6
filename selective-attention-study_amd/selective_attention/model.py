"""A decoder-only language model around the Selective Attention slot: the harness of BASELINE's
training-step (C3) and long-context prefill (C4) measurements.

It has the structure of the reference's model (src/selective_attention/model.py:41-71, 260-273,
317-418, 451-470): pre-LN blocks (no-bias LayerNorm, attention, SwiGLU MLP with hidden 8C/3),
tied input / output embeddings, N(0, 0.02) initialisation, no position signal, mean cross-entropy
over every position, cached prefill and decode. Parameter names follow the reference's, so its
state dicts load unchanged. On top of the reference it adds `prefill_chunked`, which runs a long
prompt chunk by chunk through every layer, carrying each layer's K/V cache and per-key selection
state between chunks.

Attention slots: the selective variants of `mixers.py` and "softmax" (causal SDPA, the
reference's control, model.py:74-95).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from . import mixers


@dataclass
class ModelConfig:
    """Geometry of the decoder (the reference's ModelConfig fields this harness uses,
    src/selective_attention/config.py:38-137)."""

    vocab_size: int = 50304
    n_layers: int = 24
    d_model: int = 768
    n_heads: int = 12
    context_length: int = 16384
    bias: bool = False
    dropout: float = 0.0
    mlp: str = "swiglu"
    ffn_hidden: int | None = None
    attention: str = "selective"
    layer_attention: list[str] | None = field(default=None)

    def __post_init__(self):
        if self.d_model % self.n_heads:
            raise ValueError("d_model must be divisible by n_heads")
        kinds = self.layer_kinds()
        unknown = sorted(set(kinds) - set(ATTENTION_TYPES))
        if unknown:
            raise ValueError(f"unknown attention types {unknown}; known: {ATTENTION_TYPES}")
        if self.mlp not in ("swiglu", "gelu"):
            raise ValueError("mlp must be 'swiglu' or 'gelu'")

    def layer_kinds(self) -> list[str]:
        if self.layer_attention is not None:
            if len(self.layer_attention) != self.n_layers:
                raise ValueError("layer_attention needs one entry per layer")
            return list(self.layer_attention)
        return [self.attention] * self.n_layers


ATTENTION_TYPES = ("softmax",) + mixers.MIXER_TYPES


class _AttentionBase(nn.Module):
    """q / k / v / output projections and the decode-cache plumbing shared by the attention slots."""

    def __init__(self, config: ModelConfig):
        super().__init__()
        self.c_attn = nn.Linear(config.d_model, 3 * config.d_model, bias=config.bias)
        self.c_proj = nn.Linear(config.d_model, config.d_model, bias=config.bias)
        self.resid_dropout = nn.Dropout(config.dropout)
        self.n_heads = config.n_heads
        self.d_model = config.d_model
        self.dropout = config.dropout
        self.context_length = config.context_length

    def _split_heads(self, x: Tensor, offset: int = 0) -> tuple[Tensor, Tensor, Tensor]:
        """(B, T, C) -> q, k, v (B, H, T, D). `offset` (absolute position of row 0) is unused without
        a position signal; kept for the slot interface."""
        b, t, _ = x.shape
        hd = self.d_model // self.n_heads
        qkv = self.c_attn(x).view(b, t, 3, self.n_heads, hd)
        return qkv[:, :, 0].transpose(1, 2), qkv[:, :, 1].transpose(1, 2), qkv[:, :, 2].transpose(1, 2)

    def _merge_heads(self, y: Tensor, b: int, t: int) -> Tensor:
        return self.resid_dropout(self.c_proj(y.transpose(1, 2).reshape(b, t, self.d_model)))

    def _alloc_cache(self, k: Tensor, v: Tensor, capacity: int | None = None) -> dict:
        b, h, t, d = k.shape
        cap = max(capacity if capacity is not None else self.context_length, t)
        kb, vb = k.new_zeros(b, h, cap, d), v.new_zeros(b, h, cap, d)
        kb[:, :, :t] = k
        vb[:, :, :t] = v
        return {"k": kb, "v": vb, "len": t}

    @staticmethod
    def _append_kv(cache: dict, k1: Tensor, v1: Tensor) -> int:
        t = cache["len"]
        if t >= cache["k"].shape[2]:
            raise ValueError("decode step past the cache capacity")
        cache["k"][:, :, t] = k1[:, :, 0]
        cache["v"][:, :, t] = v1[:, :, 0]
        cache["len"] = t + 1
        return t + 1


class CausalSelfAttention(_AttentionBase):
    """Causal softmax attention (SDPA): the control slot."""

    def forward(self, x: Tensor) -> Tensor:
        b, t, _ = x.shape
        q, k, v = self._split_heads(x)
        y = F.scaled_dot_product_attention(q, k, v, dropout_p=self.dropout if self.training else 0.0, is_causal=True)
        return self._merge_heads(y, b, t)

    def begin_cache(self, x: Tensor, capacity: int | None = None):
        b, t, _ = x.shape
        q, k, v = self._split_heads(x)
        y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        return self._merge_heads(y, b, t), self._alloc_cache(k, v, capacity)

    def new_cache(self, batch: int, capacity: int, device, dtype) -> dict:
        hd = self.d_model // self.n_heads
        return {"k": torch.zeros(batch, self.n_heads, capacity, hd, device=device, dtype=dtype),
                "v": torch.zeros(batch, self.n_heads, capacity, hd, device=device, dtype=dtype), "len": 0}

    def prefill_chunk(self, x: Tensor, cache: dict) -> Tensor:
        b, tc, _ = x.shape
        c0 = cache["len"]
        c1 = c0 + tc
        if c1 > cache["k"].shape[2]:
            raise ValueError("prefill chunk past the cache capacity")
        q, k, v = self._split_heads(x, offset=c0)
        cache["k"][:, :, c0:c1] = k
        cache["v"][:, :, c0:c1] = v
        cache["len"] = c1
        pos = torch.arange(c1, device=x.device)
        mask = pos[None, :] <= pos[c0:c1, None]
        y = F.scaled_dot_product_attention(q, cache["k"][:, :, :c1], cache["v"][:, :, :c1], attn_mask=mask)
        return self._merge_heads(y, b, tc)

    def step_cache(self, x1: Tensor, cache: dict) -> Tensor:
        b = x1.shape[0]
        q1, k1, v1 = self._split_heads(x1, offset=cache["len"])
        t = self._append_kv(cache, k1, v1)
        y = F.scaled_dot_product_attention(q1, cache["k"][:, :, :t], cache["v"][:, :, :t])
        return self._merge_heads(y, b, 1)


class SwiGLUMLP(nn.Module):
    def __init__(self, config: ModelConfig):
        super().__init__()
        n = config.d_model
        hidden = config.ffn_hidden if config.ffn_hidden is not None else (8 * n) // 3
        self.gate_proj = nn.Linear(n, hidden, bias=config.bias)
        self.up_proj = nn.Linear(n, hidden, bias=config.bias)
        self.down_proj = nn.Linear(hidden, n, bias=config.bias)
        self.dropout = nn.Dropout(config.dropout)

    def forward(self, x: Tensor) -> Tensor:
        return self.dropout(self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x)))


class GELUMLP(nn.Module):
    def __init__(self, config: ModelConfig):
        super().__init__()
        n = config.d_model
        hidden = config.ffn_hidden if config.ffn_hidden is not None else 4 * n
        self.c_fc = nn.Linear(n, hidden, bias=config.bias)
        self.c_proj = nn.Linear(hidden, n, bias=config.bias)
        self.dropout = nn.Dropout(config.dropout)

    def forward(self, x: Tensor) -> Tensor:
        return self.dropout(self.c_proj(F.gelu(self.c_fc(x))))


def attention_classes() -> dict:
    """Slot registry: attention type name -> factory(config) (reference model.py:306-314)."""
    reg = {"softmax": CausalSelfAttention}
    reg.update(mixers.MIXER_CLASSES)
    return reg


class Block(nn.Module):
    def __init__(self, config: ModelConfig, kind: str):
        super().__init__()
        self.ln_1 = nn.LayerNorm(config.d_model, bias=config.bias)
        self.attn = attention_classes()[kind](config)
        self.ln_2 = nn.LayerNorm(config.d_model, bias=config.bias)
        self.mlp = SwiGLUMLP(config) if config.mlp == "swiglu" else GELUMLP(config)

    def forward(self, x: Tensor) -> Tensor:
        x = x + self.attn(self.ln_1(x))
        return x + self.mlp(self.ln_2(x))

    def begin_cache(self, x: Tensor, capacity: int | None = None):
        y, cache = self.attn.begin_cache(self.ln_1(x), capacity)
        x = x + y
        return x + self.mlp(self.ln_2(x)), cache

    def prefill_chunk(self, x: Tensor, cache: dict) -> Tensor:
        x = x + self.attn.prefill_chunk(self.ln_1(x), cache)
        return x + self.mlp(self.ln_2(x))

    def step_cache(self, x1: Tensor, cache: dict) -> Tensor:
        x1 = x1 + self.attn.step_cache(self.ln_1(x1), cache)
        return x1 + self.mlp(self.ln_2(x1))


class SelectiveLM(nn.Module):
    """Decoder-only LM with tied embeddings. forward(idx, targets=None) -> (logits, loss): with
    targets, full-sequence logits and mean cross-entropy (ignore_index -100); without, the
    last position's logits."""

    def __init__(self, config: ModelConfig):
        super().__init__()
        self.config = config
        self.transformer = nn.ModuleDict({
            "wte": nn.Embedding(config.vocab_size, config.d_model),
            "drop": nn.Dropout(config.dropout),
            "h": nn.ModuleList([Block(config, kind) for kind in config.layer_kinds()]),
            "ln_f": nn.LayerNorm(config.d_model, bias=config.bias),
        })
        self.lm_head = nn.Linear(config.d_model, config.vocab_size, bias=False)
        self.transformer.wte.weight = self.lm_head.weight
        for m in self.modules():
            if isinstance(m, (nn.Linear, nn.Embedding)):
                nn.init.normal_(m.weight, mean=0.0, std=0.02)
                if getattr(m, "bias", None) is not None:
                    nn.init.zeros_(m.bias)

    def num_parameters(self) -> int:
        return sum(p.numel() for p in self.parameters())

    def _check_len(self, t: int) -> None:
        if t > self.config.context_length:
            raise ValueError(f"sequence length {t} exceeds context_length {self.config.context_length}")

    def forward(self, idx: Tensor, targets: Tensor | None = None):
        self._check_len(idx.shape[1])
        x = self.transformer.drop(self.transformer.wte(idx))
        for block in self.transformer.h:
            x = block(x)
        x = self.transformer.ln_f(x)
        if targets is None:
            return self.lm_head(x[:, -1:]), None
        logits = self.lm_head(x)
        loss = F.cross_entropy(logits.reshape(-1, logits.shape[-1]), targets.reshape(-1), ignore_index=-100)
        return logits, loss

    def prefill(self, idx: Tensor, capacity: int | None = None):
        """Single-shot prompt pass: last-position logits and per-layer caches."""
        x = self.transformer.drop(self.transformer.wte(idx))
        caches = []
        for block in self.transformer.h:
            x, cache = block.begin_cache(x, capacity)
            caches.append(cache)
        return self.lm_head(self.transformer.ln_f(x)[:, -1:]), caches

    def prefill_chunked(self, idx: Tensor, chunk: int, capacity: int | None = None):
        """Prompt pass in chunks of `chunk` tokens through all layers, each layer carrying its K/V
        and per-key selection state between chunks; same result as `prefill` up to fp32 rounding.
        Returns last-position logits and per-layer caches (usable by decode_step)."""
        b, t = idx.shape
        cap = max(capacity or 0, t)
        dtype = torch.get_autocast_dtype(idx.device.type) if torch.is_autocast_enabled(idx.device.type) else \
            self.lm_head.weight.dtype
        caches = [block.attn.new_cache(b, cap, idx.device, dtype) for block in self.transformer.h]
        last = None
        for c0 in range(0, t, chunk):
            x = self.transformer.drop(self.transformer.wte(idx[:, c0:c0 + chunk]))
            for block, cache in zip(self.transformer.h, caches):
                x = block.prefill_chunk(x, cache)
            last = x[:, -1:]
        return self.lm_head(self.transformer.ln_f(last)), caches

    def decode_step(self, token: Tensor, position: int, caches) -> Tensor:
        """One cached step: (B, 1) token ids -> (B, 1, vocab) logits."""
        del position   # no position signal
        x = self.transformer.drop(self.transformer.wte(token))
        for block, cache in zip(self.transformer.h, caches):
            x = block.step_cache(x, cache)
        return self.lm_head(self.transformer.ln_f(x))
