"""A decoder-only language model around the Selective Attention slot: the harness of BASELINE's
training-step (C3) and long-context prefill (C4) measurements.

Architecture (the reference's 16K study model, src/selective_attention/model.py:342-418 and
configs/scale_16384/all_selective_nope_bos.yaml): token embedding with no position signal, pre-norm
residual blocks (LayerNorm without bias -> attention slot; LayerNorm -> SwiGLU feed-forward of
width 8C/3), a final LayerNorm, and an output head tied to the embedding; weights N(0, 0.02); the
loss is the mean cross-entropy over every position. The module and parameter names are the
reference's (transformer.wte / h.N.ln_1 / attn.c_attn / ... / lm_head), so its state dicts load.

Generation keeps one cache per layer (slot.py): `prefill` runs the prompt in one pass, and
`prefill_chunked` in chunks through all layers, each layer's slot carrying its keys, values and
per-key selection state between chunks; `decode_step` then adds one token at a time.

Attention slots: the selective variants of `mixers.py` and "softmax" (causal SDPA, the reference's
control slot).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from . import mixers
from .slot import AttentionSlot


@dataclass
class ModelConfig:
    """Decoder geometry (the fields of the reference's ModelConfig that this harness uses,
    src/selective_attention/config.py:38-137). Defaults: the reference's 209M model."""

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
    layer_attention: list[str] | None = None

    def __post_init__(self):
        if self.d_model % self.n_heads:
            raise ValueError("d_model must be divisible by n_heads")
        unknown = sorted(set(self.layer_kinds()) - set(ATTENTION_TYPES))
        if unknown:
            raise ValueError(f"unknown attention types {unknown}; known: {ATTENTION_TYPES}")
        if self.mlp != "swiglu":
            raise ValueError("this harness builds the study model's SwiGLU feed-forward only (mlp='swiglu')")

    def layer_kinds(self) -> list[str]:
        """The attention type of every layer."""
        kinds = [self.attention] * self.n_layers if self.layer_attention is None else list(self.layer_attention)
        if len(kinds) != self.n_layers:
            raise ValueError("layer_attention needs one entry per layer")
        return kinds


class CausalSelfAttention(AttentionSlot):
    """Causal softmax attention through SDPA: the control slot."""

    def _sdpa(self, q: Tensor, keys: Tensor, vals: Tensor, first: int = 0) -> Tensor:
        """Queries at positions [first, first + n) over keys [0, first + n)."""
        n, t = q.shape[2], keys.shape[2]
        p = self.dropout if self.training else 0.0
        if first == 0 and n == t:
            return F.scaled_dot_product_attention(q, keys, vals, dropout_p=p, is_causal=True)
        allowed = torch.arange(t, device=q.device)[None, :] <= torch.arange(first, first + n, device=q.device)[:, None]
        return F.scaled_dot_product_attention(q, keys, vals, attn_mask=allowed, dropout_p=p)

    def forward(self, x: Tensor) -> Tensor:
        return self.emit(self._sdpa(*self.project(x)))

    def begin_cache(self, x: Tensor, capacity: int | None = None):
        q, k, v = self.project(x)
        return self.emit(self._sdpa(q, k, v)), self.prompt_cache(k, v, capacity)

    def prefill_chunk(self, x: Tensor, cache: dict) -> Tensor:
        q, k, v = self.project(x)
        c0, c1 = self.cache_put(cache, k, v)
        return self.emit(self._sdpa(q, cache["k"][:, :, :c1], cache["v"][:, :, :c1], c0))

    def step_cache(self, x1: Tensor, cache: dict) -> Tensor:
        return self.prefill_chunk(x1, cache)


class GatedMLP(nn.Module):
    """SwiGLU feed-forward, hidden width 8C/3 unless the config sets ffn_hidden: the product of
    silu(gate_proj x) and up_proj x, projected back by down_proj."""

    def __init__(self, config: ModelConfig):
        super().__init__()
        width = config.d_model
        hidden = (8 * width) // 3 if config.ffn_hidden is None else config.ffn_hidden
        self.gate_proj, self.up_proj = (nn.Linear(width, hidden, bias=config.bias) for _ in range(2))
        self.down_proj = nn.Linear(hidden, width, bias=config.bias)
        self.dropout = nn.Dropout(config.dropout)

    def forward(self, x: Tensor) -> Tensor:
        gated = F.silu(self.gate_proj(x)) * self.up_proj(x)
        return self.dropout(self.down_proj(gated))


def attention_classes() -> dict:
    """Slot registry: attention type name -> factory(config) (reference model.py:306-314)."""
    return {"softmax": CausalSelfAttention, **mixers.MIXER_CLASSES}


ATTENTION_TYPES = tuple(attention_classes())


class Block(nn.Module):
    """Pre-norm residual block: x + attn(ln_1 x), then + mlp(ln_2 .). The cached forms run the same
    residual stream through the slot's prefill / chunk / decode operation."""

    def __init__(self, config: ModelConfig, kind: str):
        super().__init__()
        self.ln_1 = nn.LayerNorm(config.d_model, bias=config.bias)
        self.attn = attention_classes()[kind](config)
        self.ln_2 = nn.LayerNorm(config.d_model, bias=config.bias)
        self.mlp = GatedMLP(config)

    def _through(self, x: Tensor, mixed: Tensor) -> Tensor:
        h = x + mixed
        return h + self.mlp(self.ln_2(h))

    def forward(self, x: Tensor) -> Tensor:
        return self._through(x, self.attn(self.ln_1(x)))

    def begin_cache(self, x: Tensor, capacity: int | None = None):
        mixed, cache = self.attn.begin_cache(self.ln_1(x), capacity)
        return self._through(x, mixed), cache

    def prefill_chunk(self, x: Tensor, cache: dict) -> Tensor:
        return self._through(x, self.attn.prefill_chunk(self.ln_1(x), cache))

    def step_cache(self, x1: Tensor, cache: dict) -> Tensor:
        return self._through(x1, self.attn.step_cache(self.ln_1(x1), cache))


class SelectiveLM(nn.Module):
    """Decoder-only LM. forward(idx, targets=None) -> (logits, loss): with targets, every position's
    logits and the mean cross-entropy (ignore_index -100); without, the last position's logits."""

    def __init__(self, config: ModelConfig):
        super().__init__()
        self.config = config
        layers = nn.ModuleList(Block(config, kind) for kind in config.layer_kinds())
        self.transformer = nn.ModuleDict(dict(
            wte=nn.Embedding(config.vocab_size, config.d_model), drop=nn.Dropout(config.dropout), h=layers,
            ln_f=nn.LayerNorm(config.d_model, bias=config.bias)))
        self.lm_head = nn.Linear(config.d_model, config.vocab_size, bias=False)
        self.lm_head.weight = self.transformer.wte.weight   # one matrix: embedding and output head
        self.apply(self._init)

    @staticmethod
    def _init(module: nn.Module) -> None:
        if isinstance(module, (nn.Linear, nn.Embedding)):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)
        if isinstance(module, nn.Linear) and module.bias is not None:
            nn.init.zeros_(module.bias)

    def num_parameters(self) -> int:
        return sum(p.numel() for p in self.parameters())

    def _embed(self, idx: Tensor) -> Tensor:
        return self.transformer.drop(self.transformer.wte(idx))

    def _head(self, x: Tensor) -> Tensor:
        return self.lm_head(self.transformer.ln_f(x))

    def forward(self, idx: Tensor, targets: Tensor | None = None):
        if idx.shape[1] > self.config.context_length:
            raise ValueError(f"sequence length {idx.shape[1]} exceeds context_length {self.config.context_length}")
        x = self._embed(idx)
        for block in self.transformer.h:
            x = block(x)
        if targets is None:
            return self._head(x[:, -1:]), None
        logits = self._head(x)
        return logits, F.cross_entropy(logits.flatten(0, 1), targets.flatten(), ignore_index=-100)

    def prefill(self, idx: Tensor, capacity: int | None = None):
        """The prompt in one pass: last-position logits and one cache per layer."""
        x, caches = self._embed(idx), []
        for block in self.transformer.h:
            x, cache = block.begin_cache(x, capacity)
            caches.append(cache)
        return self._head(x[:, -1:]), caches

    def prefill_chunked(self, idx: Tensor, chunk: int, capacity: int | None = None):
        """The prompt in chunks of `chunk` tokens through all layers, each layer carrying its keys,
        values and per-key selection state from chunk to chunk; equal to `prefill` up to fp32
        rounding. Returns last-position logits and the caches (usable by decode_step)."""
        b, t = idx.shape
        device = idx.device
        dtype = (torch.get_autocast_dtype(device.type) if torch.is_autocast_enabled(device.type)
                 else self.lm_head.weight.dtype)
        caches = [block.attn.new_cache(b, max(t, capacity or 0), device, dtype) for block in self.transformer.h]
        x = None
        for start in range(0, t, chunk):
            x = self._embed(idx[:, start:start + chunk])
            for block, cache in zip(self.transformer.h, caches):
                x = block.prefill_chunk(x, cache)
        return self._head(x[:, -1:]), caches

    def decode_step(self, token: Tensor, position: int, caches) -> Tensor:
        """One cached step: (B, 1) token ids -> (B, 1, vocab) logits. `position` is unused: the model
        has no position signal."""
        x = self._embed(token)
        for block, cache in zip(self.transformer.h, caches):
            x = block.step_cache(x, cache)
        return self._head(x)
