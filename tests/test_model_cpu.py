"""The decoder harness and the SelectiveAttention slot on the CPU (reference tests/test_selective_model.py,
tests/test_selective_perhead.py). On CPU tensors the layers run the plain listing, as the reference's
do; the kernel path of the same layers is tested on the GPU (test_model_gpu.py)."""

from __future__ import annotations

import pytest
import torch

from oracle import sa_oracle
from selective_attention import mixers
from selective_attention.model import ATTENTION_TYPES, ModelConfig, SelectiveLM, attention_classes


def _tiny(attention="selective", layers=2, **kw):
    cfg = ModelConfig(vocab_size=97, n_layers=layers, d_model=64, n_heads=4, context_length=64, attention=attention,
                      **kw)
    torch.manual_seed(0)
    model = SelectiveLM(cfg).double()
    for block in model.transformer.h:
        block.attn.use_kernel = False
    return model.eval()


def test_registry_names_match_the_reference():
    """reference mixers.py:21-32, tests/test_selective_model.py:24-27"""
    assert mixers.MIXER_TYPES == ("selective", "selective_x16", "selective_perhead")
    assert set(attention_classes()) == {"softmax", *mixers.MIXER_TYPES}
    assert set(ATTENTION_TYPES) == set(attention_classes())
    with pytest.raises(ValueError, match="unknown attention"):
        ModelConfig(attention="dilution")


def test_mixed_stack_builds():
    """Layers of different attention types in one stack (reference tests/test_selective_model.py:
    36-40; its "dilution" layer is not part of this package)."""
    model = _tiny(layers=3, layer_attention=["selective", "softmax", "selective_x16"])
    assert [type(b.attn).__name__ for b in model.transformer.h] == [
        "SelectiveAttention", "CausalSelfAttention", "SelectiveAttention"]
    assert model.transformer.h[2].attn.exempt == 16
    idx = torch.randint(0, 97, (2, 40))
    logits, loss = model(idx, idx)
    assert logits.shape == (2, 40, 97) and torch.isfinite(loss)


def test_parameter_counts():
    """208,540,416 is the reference run record's count for its 16K model
    (runs/scale_16384/all_selective_nope_bos_seed1337/metrics.jsonl:1); d1024/16H is BASELINE's
    literal geometry. Selective attention adds no parameters over softmax attention."""
    with torch.device("meta"):
        assert SelectiveLM(ModelConfig()).num_parameters() == 208_540_416
        assert SelectiveLM(ModelConfig(d_model=1024, n_heads=16)).num_parameters() == 353_502_208
        assert (SelectiveLM(ModelConfig(n_layers=2)).num_parameters()
                == SelectiveLM(ModelConfig(n_layers=2, attention="softmax")).num_parameters())


def test_state_dict_names_follow_the_reference():
    keys = set(SelectiveLM(ModelConfig(n_layers=1, d_model=64, n_heads=4, vocab_size=50)).state_dict())
    assert keys == {"transformer.wte.weight", "lm_head.weight", "transformer.ln_f.weight",
                    "transformer.h.0.ln_1.weight", "transformer.h.0.ln_2.weight",
                    "transformer.h.0.attn.c_attn.weight", "transformer.h.0.attn.c_proj.weight",
                    "transformer.h.0.mlp.gate_proj.weight", "transformer.h.0.mlp.up_proj.weight",
                    "transformer.h.0.mlp.down_proj.weight"}


def test_layer_matches_the_oracle():
    """One SelectiveAttention layer == projections around oracle.attention."""
    model = _tiny()
    layer = model.transformer.h[0].attn
    x = torch.randn(2, 30, 64, dtype=torch.float64)
    q, k, v = layer.project(x)
    want = layer.emit(sa_oracle.attention(q, k, v))
    torch.testing.assert_close(layer(x), want)


@pytest.mark.parametrize("attention", ["selective", "selective_x16", "selective_perhead"])
def test_cached_decode_equals_full_forward(attention):
    """Prefill then decode steps give the full forward's logits (reference
    tests/test_selective_model.py:42-53, test_selective_perhead.py:32-51)."""
    model = _tiny(attention)
    idx = torch.randint(0, 97, (2, 40))
    with torch.no_grad():
        full = model.transformer.ln_f(_hidden(model, idx))
        full_logits = model.lm_head(full)
        logits, caches = model.prefill(idx[:, :25], capacity=40)
        torch.testing.assert_close(logits[:, 0], full_logits[:, 24])
        for t in range(25, 40):
            step = model.decode_step(idx[:, t:t + 1], t, caches)
            torch.testing.assert_close(step[:, 0], full_logits[:, t])


def _hidden(model, idx):
    x = model.transformer.wte(idx)
    for block in model.transformer.h:
        x = block(x)
    return x


def test_per_head_layer_is_each_head_alone():
    """selective_perhead == every head as its own one-head sequence (reference mixers.py:76-84)."""
    model = _tiny("selective_perhead")
    layer = model.transformer.h[0].attn
    x = torch.randn(1, 20, 64, dtype=torch.float64)
    q, k, v = layer.project(x)
    torch.testing.assert_close(layer._attend(q, k, v)[0], sa_oracle.per_head(q, k, v))


def test_cpu_tensors_route_to_the_listing():
    """With use_kernel on (the default), CPU tensors run the listing, as in the reference
    (mixers.py:73-74, 87-98): the same outputs and gradients as use_kernel = False."""
    torch.manual_seed(4)
    idx = torch.randint(0, 97, (2, 33))
    on, off = _tiny(), _tiny()
    for block in on.transformer.h:
        block.attn.use_kernel = True
    on.train(), off.train()
    _, l_on = on(idx[:, :-1], idx[:, 1:])
    _, l_off = off(idx[:, :-1], idx[:, 1:])
    l_on.backward(), l_off.backward()
    torch.testing.assert_close(l_on, l_off, rtol=0, atol=0)
    for (name, a), (_, b) in zip(on.named_parameters(), off.named_parameters()):
        torch.testing.assert_close(a.grad, b.grad, rtol=0, atol=0, msg=lambda m: f"{name}: {m}")


@pytest.mark.parametrize("attention,chunk", [("selective", 7), ("selective_perhead", 16), ("selective_x16", 5)])
def test_chunked_prefill_equals_single_shot_on_cpu(attention, chunk):
    """prefill_chunked (each layer's K/V and selection state carried between chunks) == prefill,
    on the listing's chunk form."""
    model = _tiny(attention)
    idx = torch.randint(0, 97, (2, 37))
    with torch.no_grad():
        a, ca = model.prefill(idx, capacity=40)
        b, cb = model.prefill_chunked(idx, chunk, capacity=40)
        torch.testing.assert_close(a, b)
        for x, y in zip(ca, cb):
            torch.testing.assert_close(x["selected"][:, :, :37], y["selected"][:, :, :37])
        torch.testing.assert_close(model.decode_step(idx[:, -1:], 37, ca), model.decode_step(idx[:, -1:], 37, cb))


def test_registry_factories_build_the_variants():
    cfg = ModelConfig(vocab_size=50, n_layers=1, d_model=64, n_heads=4, context_length=32)
    layers = {name: make(cfg) for name, make in mixers.MIXER_CLASSES.items()}
    assert (layers["selective"].exempt, layers["selective"].groups) == (1, 1)
    assert (layers["selective_x16"].exempt, layers["selective_x16"].groups) == (16, 1)
    assert (layers["selective_perhead"].exempt, layers["selective_perhead"].groups) == (1, 4)
    with pytest.raises(ValueError, match="swiglu"):
        ModelConfig(mlp="gelu")


def test_training_loss_and_backward_on_cpu_listing():
    model = _tiny().train()
    idx = torch.randint(0, 97, (2, 33))
    _, loss = model(idx[:, :-1], idx[:, 1:])
    loss.backward()
    assert torch.isfinite(loss) and all(torch.isfinite(p.grad).all() for p in model.parameters())
