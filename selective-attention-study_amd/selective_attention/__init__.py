"""Selective Attention (Leviathan, Kalman, Matias; ICLR 2025) on MI355X HIP kernels.

Same exports as the reference package (reference src/selective_attention/__init__.py:3-17), plus
the chunked-prefill, cached-decode and packed-projection entry points.
"""

from .kernels import (
    HAS_HIP,
    HAS_TRITON,
    selective_attention,
    selective_attention_decode,
    selective_attention_forward,
    selective_attention_prefill,
    selective_attention_qkv,
    selective_attention_reference,
    selective_logits,
)

__all__ = [
    "HAS_HIP",
    "HAS_TRITON",
    "selective_attention",
    "selective_attention_decode",
    "selective_attention_forward",
    "selective_attention_prefill",
    "selective_attention_qkv",
    "selective_attention_reference",
    "selective_logits",
]
