"""The attention slot under torch.compile (the reference trains compiled, train.py:557-562): with
fullgraph=True the whole model traces through the kernels' custom ops and their fake (meta) kernels
without a graph break, and the compiled step equals the eager one. The "aot_eager" backend runs the
traced forward and backward graphs as they are (no code generation), which is what checks the
boundary."""

from __future__ import annotations

import pytest
import torch

from selective_attention import harness, kernels
from selective_attention.model import ModelConfig, SelectiveLM

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("attention", ["selective", "selective_perhead"])
def test_slot_under_torch_compile_equals_eager(cuda, attention):
    print(f"case compile {attention}", flush=True)
    torch._dynamo.reset()
    cfg = ModelConfig(vocab_size=211, n_layers=2, d_model=256, n_heads=4, context_length=320, attention=attention)
    torch.manual_seed(0)
    eager = SelectiveLM(cfg).to(cuda)
    twin = SelectiveLM(cfg).to(cuda)
    twin.load_state_dict(eager.state_dict())
    compiled = torch.compile(twin, backend="aot_eager", fullgraph=True)
    idx, tgt = harness.synthetic_batch(2, 300, cuda)
    idx, tgt = idx % 211, tgt % 211
    losses = []
    for model in (eager, compiled):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            _, loss = model(idx, tgt)
        loss.backward()
        losses.append(loss.detach())
    torch.testing.assert_close(losses[1], losses[0], rtol=1e-5, atol=1e-5)
    for (name, a), (_, b) in zip(eager.named_parameters(), twin.named_parameters()):
        # the attention gradients repeat bit for bit, but torch's own kernels elsewhere in the model
        # (the tied embedding's gradient among them) may sum in a varying order
        torch.testing.assert_close(b.grad, a.grad, rtol=2e-2, atol=1e-4, msg=lambda m: f"{name}: {m}")


def test_custom_ops_pass_opcheck(cuda):
    """torch.library.opcheck: schema, fake kernel and real kernel agree on a small bf16 call."""
    g = torch.Generator(device=cuda).manual_seed(1)
    q, k, v = (torch.randn(1, 2, 70, 64, device=cuda, generator=g).bfloat16() for _ in range(3))
    torch.library.opcheck(torch.ops.selective_attention.forward.default, (q, k, v, 0.125, 1, 0, 0, 0),
                          test_utils=("test_schema", "test_faketensor"))
    out, rmax, rden, carry, _ = torch.ops.selective_attention.forward(q, k, v, 0.125, 1, 0, 0, 0)
    torch.library.opcheck(torch.ops.selective_attention.backward.default,
                          (q, k, v, out, q, rmax, rden, carry, 0.125, 1, 0, True),
                          test_utils=("test_schema", "test_faketensor"))
    assert kernels.HAS_HIP
