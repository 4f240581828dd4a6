"""BASELINE's configurations at their full sizes, checked through properties that do not need (T x T)
tensors (reference tests/test_selective_kernels.py:310-345, tests/test_selective_model.py:91-100):

  C4  one attention layer's prefill of 131,072 tokens in 8 chunks of 16,384 (B=1, H=16, D=64,
      bf16): chunked == single shot, the last 1000 queries against the oracle's chunk-summed tail form,
      the carried per-key state against the tail's totals
  C3  one training step of the 24-layer d1024 / 16-head decoder at 1 x 16,384 tokens under bf16
      autocast: finite loss and gradients; chunked model prefill == single-shot prefill
  the forward past the int32 offset limit (T = 270,000, where CARRY's block x T index passes 2^31)

The oracle's tail runs in float64 on the GPU box's GPU here (plain torch products on the oracle's
own formulation; at these lengths its CPU form takes minutes).
"""

from __future__ import annotations

import pytest
import torch

from oracle import sa_oracle
from selective_attention import harness, kernels
from selective_attention.model import ModelConfig, SelectiveLM

pytestmark = pytest.mark.gpu


def test_c4_chunked_prefill_131072(cuda):
    b, h, t, d, chunk = 1, 16, 131072, 64, 16384
    print(f"case C4 prefill T={t} chunk={chunk}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(404)
    q, k, v = (torch.randn(b, h, t, d, device=cuda, generator=g).bfloat16() for _ in range(3))
    state = torch.zeros(b, t, device=cuda)
    outs = []
    for c0 in range(0, t, chunk):
        c1 = c0 + chunk
        outs.append(kernels.selective_attention_prefill(q[:, :, c0:c1], k[:, :, :c1], v[:, :, :c1], state, c0))
    got = torch.cat(outs, dim=2)
    del outs
    full, aux = kernels.selective_attention_forward(q, k, v, return_aux=True)
    rel = ((got - full).abs().max() / full.abs().max()).item()
    print(f"C4 chunked vs single shot: rel {rel:.2e}", flush=True)
    assert rel <= 1e-2
    del full
    rows, want, total = sa_oracle.tail(q.double(), k.double(), v.double(), 1000, chunk=4096)
    err = (got[:, :, rows].double() - want).abs().max().item()
    srel = ((state.double() - total).abs().max() / total.abs().max()).item()
    arel = ((aux["selected_total"].double() - total).abs().max() / total.abs().max()).item()
    print(f"C4 tail max-abs {err:.2e}, state rel {srel:.2e}, single-shot totals rel {arel:.2e}", flush=True)
    assert err < 2e-2
    assert srel < 1e-4 and arel < 1e-4


def test_forward_past_the_int32_offset_limit(cuda):
    """CARRY is (B, T/32, T): block index x T passes 2^31 from T ~ 262K. A forward at T = 270,000
    (9.1 GB of CARRY) matches the oracle in its last queries (reference
    tests/test_selective_kernels.py:333-345: fp32 "ieee", H=2, D=16, the last 1000 queries)."""
    seq = 270_000
    print(f"case int32 offsets T={seq}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(31)
    q, k, v = (torch.randn(1, 2, seq, 16, device=cuda, generator=g) for _ in range(3))
    got, aux = kernels.selective_attention_forward(q, k, v, dot_precision="ieee", return_aux=True)
    rows, want, total = sa_oracle.tail(q.double(), k.double(), v.double(), 1000, chunk=8192)
    torch.testing.assert_close(got[:, :, rows].double(), want, atol=2e-4, rtol=2e-4)
    torch.testing.assert_close(aux["selected_total"].double(), total, atol=1e-2, rtol=1e-3)


def test_bf16_fwd_bwd_past_the_int32_offset_limit(cuda):
    """The bf16 kernels at head dim 64 (direct loads into LDS) at T = 270,000, where CARRY's and the
    checkpoint planes' element offsets pass 2^31: the last queries against the oracle's tail, finite
    gradients, and the last key's dV, which only the last query attends: P[T-1, T-1] dO[T-1]."""
    seq, heads = 270_000, 2
    print(f"case bf16 fwd+bwd T={seq}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(32)
    q, k, v = (torch.randn(1, heads, seq, 64, device=cuda, generator=g).bfloat16().requires_grad_(True)
               for _ in range(3))
    out = kernels.selective_attention(q, k, v)
    dout = torch.randn(out.shape, device=cuda, generator=g)
    dq, dk, dv = torch.autograd.grad(out, (q, k, v), dout)
    rows, want, total = sa_oracle.tail(q.detach().double(), k.detach().double(), v.detach().double(), 64,
                                       chunk=8192)
    err = (out[:, :, rows].detach().double() - want).abs().max().item()
    print(f"tail max-abs {err:.2e}", flush=True)
    assert err < 2e-2
    assert all(torch.isfinite(x).all() for x in (dq, dk, dv))
    # the last row's weight on its own key: its logits less the history every key gathered from the
    # earlier queries (the totals less the last query's own selection)
    qd, kd = q.detach().double(), k.detach().double()
    lg = sa_oracle.raw_logits(qd[:, :, -1:], kd)                          # (1, H, 1, T)
    own = sa_oracle.selection(qd[:, :, -1:], kd, 1, q_offset=seq - 1)     # (1, 1, T)
    hist = total - own[:, 0]                                              # (1, T)
    p = torch.softmax(lg - hist[:, None, None, :], dim=-1)[..., -1]       # (1, H, 1)
    want_dv = p[..., None] * dout[:, :, -1:].double()
    got_dv = dv[:, :, -1:].double()
    scale = want_dv.abs().max().item()
    rel = ((got_dv - want_dv).abs().max() / scale).item()
    print(f"last-key dV rel {rel:.2e}", flush=True)
    assert rel < 2e-2


def test_c3_training_step_d1024_16384(cuda):
    """C3: one full training step (forward, backward, clipping, fused AdamW) of the 24-layer
    d1024 / 16-head decoder on 1 x 16,384 tokens under bf16 autocast: the loss and every gradient
    are finite, over two steps."""
    print("case C3 train step d1024 T=16384", flush=True)
    cfg = ModelConfig(n_layers=24, context_length=16384, **harness.GEOMETRIES["d1024"])
    torch.manual_seed(0)
    model = SelectiveLM(cfg).to(cuda).train()
    assert model.num_parameters() == 353_502_208
    opt = torch.optim.AdamW(model.parameters(), lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, fused=True)
    idx, tgt = harness.synthetic_batch(1, 16384, cuda)
    losses = []
    for _ in range(2):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            _, loss = model(idx, tgt)
        loss.backward()
        assert torch.isfinite(loss)
        bad = [n for n, p in model.named_parameters() if p.grad is not None and not torch.isfinite(p.grad).all()]
        assert not bad, bad[:5]
        assert all(p.grad is not None for p in model.parameters())
        torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
        opt.step()
        opt.zero_grad(set_to_none=True)
        losses.append(loss.item())
    print(f"C3 losses {losses}", flush=True)


def test_c3_geometry_chunked_prefill_equals_single_shot(cuda):
    """The model's chunked prefill (each layer's K/V and per-key selection state carried between
    chunks) equals its single-shot prefill at the d1024 / 16-head geometry in bf16."""
    print("case C3-geometry chunked prefill", flush=True)
    cfg = ModelConfig(n_layers=2, context_length=4096, **harness.GEOMETRIES["d1024"])
    torch.manual_seed(1)
    model = SelectiveLM(cfg).to(cuda, torch.bfloat16).eval()
    idx, _ = harness.synthetic_batch(1, 4096, cuda, seed=3)
    with torch.no_grad():
        a, ca = model.prefill(idx)
        bb, cb = model.prefill_chunked(idx, 1024)
    rel = ((a.float() - bb.float()).abs().max() / a.float().abs().max()).item()
    assert rel < 2e-2, rel
    for x, y in zip(ca, cb):
        s = x["selected"][:, :, :4096]
        assert ((s - y["selected"][:, :, :4096]).abs().max() / s.abs().max()).item() < 2e-2
