"""The decoder harness on the GPU: the kernel path inside the model against the listing path (reference
tests/test_selective_model.py:56-100, test_selective_perhead.py:54-77), cached and chunked prefill
against the full forward, and a bf16 autocast training step."""

from __future__ import annotations

import pytest
import torch

from selective_attention import harness
from selective_attention.model import ModelConfig, SelectiveLM

pytestmark = pytest.mark.gpu


def _pair(attention, cuda, layers=2, d_model=128, heads=4):
    cfg = ModelConfig(vocab_size=211, n_layers=layers, d_model=d_model, n_heads=heads, context_length=256,
                      attention=attention)
    torch.manual_seed(0)
    a = SelectiveLM(cfg).to(cuda)
    b = SelectiveLM(cfg).to(cuda)
    b.load_state_dict(a.state_dict())
    for block in b.transformer.h:
        block.attn.use_kernel = False
    return a, b


@pytest.mark.parametrize("attention", ["selective", "selective_x16", "selective_perhead"])
def test_kernel_model_matches_listing_model(cuda, attention):
    """fp32 model: loss and every parameter gradient through the kernels match the listing."""
    print(f"case model parity {attention}", flush=True)
    ker, ref = _pair(attention, cuda)
    idx, tgt = harness.synthetic_batch(2, 130, cuda)
    idx, tgt = idx % 211, tgt % 211
    _, lk = ker(idx, tgt)
    _, lr = ref(idx, tgt)
    lk.backward()
    lr.backward()
    torch.testing.assert_close(lk, lr, atol=1e-5, rtol=1e-5)
    for (name, pk), (_, pr) in zip(ker.named_parameters(), ref.named_parameters()):
        torch.testing.assert_close(pk.grad, pr.grad, atol=2e-5, rtol=1e-3, msg=lambda m: f"{name}: {m}")


@pytest.mark.parametrize("attention", ["selective", "selective_perhead"])
def test_kernel_prefill_then_decode_equals_full_forward(cuda, attention):
    """reference tests/test_selective_model.py:74-88"""
    ker, _ = _pair(attention, cuda)
    ker.eval()
    idx, _ = harness.synthetic_batch(2, 90, cuda)
    idx = idx % 211
    with torch.no_grad():
        x = ker.transformer.wte(idx)
        for block in ker.transformer.h:
            x = block(x)
        full = ker.lm_head(ker.transformer.ln_f(x))
        logits, caches = ker.prefill(idx[:, :70], capacity=90)
        torch.testing.assert_close(logits[:, 0], full[:, 69], atol=1e-4, rtol=1e-4)
        for t in range(70, 90):
            step = ker.decode_step(idx[:, t:t + 1], t, caches)
            torch.testing.assert_close(step[:, 0], full[:, t], atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("attention,chunk", [("selective", 32), ("selective", 50), ("selective_perhead", 64),
                                             ("selective_x16", 7)])
def test_chunked_prefill_equals_single_shot(cuda, attention, chunk):
    """prefill_chunked (per-layer K/V and selection state carried across chunks) == prefill."""
    print(f"case chunked prefill {attention} chunk={chunk}", flush=True)
    ker, _ = _pair(attention, cuda)
    ker.eval()
    idx, _ = harness.synthetic_batch(2, 160, cuda)
    idx = idx % 211
    with torch.no_grad():
        a, ca = ker.prefill(idx, capacity=200)
        b, cb = ker.prefill_chunked(idx, chunk, capacity=200)
        torch.testing.assert_close(a, b, atol=1e-4, rtol=1e-4)
        for x, y in zip(ca, cb):
            torch.testing.assert_close(x["selected"][:, :, :160], y["selected"][:, :, :160], atol=1e-3, rtol=1e-5)
        # decoding continues from either cache alike
        nxt = idx[:, -1:]
        torch.testing.assert_close(ker.decode_step(nxt, 160, ca), ker.decode_step(nxt, 160, cb), atol=1e-4,
                                   rtol=1e-4)


def test_bf16_autocast_training_step_is_finite(cuda):
    """reference tests/test_selective_model.py:91-100"""
    cfg = ModelConfig(vocab_size=50304, n_layers=2, d_model=256, n_heads=4, context_length=1024)
    torch.manual_seed(0)
    model = SelectiveLM(cfg).to(cuda)
    opt = torch.optim.AdamW(model.parameters(), lr=6e-4, betas=(0.9, 0.95), weight_decay=0.1, fused=True)
    idx, tgt = harness.synthetic_batch(1, 1024, cuda)
    for _ in range(2):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            _, loss = model(idx, tgt)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
        opt.step()
        opt.zero_grad(set_to_none=True)
        assert torch.isfinite(loss)
