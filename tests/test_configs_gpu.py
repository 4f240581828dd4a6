"""BASELINE's configurations at their full sizes, checked through properties that do not need (T x T)
tensors (reference tests/test_selective_kernels.py:310-345, tests/test_selective_model.py:91-100):

  C4  one attention layer's prefill of 131,072 tokens in 8 chunks of 16,384 (B=1, H=16, D=64,
      bf16): chunked == single shot, the last 1000 queries against the oracle's chunk-summed tail form,
      the carried per-key state against the tail's totals
  C5  per-head selection fwd+bwd at B=2, H=16, T=32,768, D=64 in bf16 on the bench's own inputs: the
      first 2048 rows == a T=2048 run bit for bit, the last rows of two sequences against the
      oracle's tail, finite gradients, the last key's dV against P[T-1, T-1] dO[T-1]
  C3  one training step of the 24-layer decoder at 1 x 16,384 tokens under bf16 autocast, at the
      reference's d768 / 12-head geometry and BASELINE's d1024 / 16-head one: finite loss and
      gradients; chunked model prefill == single-shot prefill
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
    want_dv = _last_key_dv(q.detach().double(), k.detach().double(), dout, total)
    got_dv = dv[:, :, -1:].double()
    scale = want_dv.abs().max().item()
    rel = ((got_dv - want_dv).abs().max() / scale).item()
    print(f"last-key dV rel {rel:.2e}", flush=True)
    assert rel < 2e-2


def _last_key_dv(q, k, dout, total):
    """dV of the last key, which only the last query attends: P[T-1, T-1] dO[T-1] per head, P the
    last row's softmax over its logits less the history every key gathered from the earlier queries
    (the totals less the last query's own selection). q, k (B, H, T, D) float64; total (B, T)."""
    seq = q.shape[2]
    lg = sa_oracle.raw_logits(q[:, :, -1:], k)                           # (B, H, 1, T)
    own = sa_oracle.selection(q[:, :, -1:], k, 1, q_offset=seq - 1)      # (B, 1, T)
    hist = total - own[:, 0]                                             # (B, T)
    p = torch.softmax(lg - hist[:, None, None, :], dim=-1)[..., -1]      # (B, H, 1)
    return p[..., None] * dout[:, :, -1:].double()


def test_c5_per_head_full_size(cuda):
    """C5 at its full size on the bench's own inputs (harness.perhead_rate: q, k, v, dO ~ N(0,1) from
    seed 5 on the GPU, k scaled by 2 on a random 10% of key positions, each head its own one-head
    sequence): the one-pass selection carry over 32 sequences (4.3 GB of CARRY), the one-head forward
    and the one-head backward instances at T = 32768. The first 2048 output rows equal a T=2048 run
    bit for bit (causality); the last 64 rows of two sequences and their selection totals agree with
    the oracle's tail (float64 on the GPU); the gradients are finite and in bf16; the last key's dV
    equals P[T-1, T-1] dO[T-1] (reference tests/test_selective_perhead.py:55-77 checks per-head
    selection against each head alone, here at the configuration's own length)."""
    b, h, t, d = 2, 16, 32768, 64
    print(f"case C5 per-head full size B={b} H={h} T={t}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(5)
    q, k, v, do = (torch.randn(b, h, t, d, device=cuda, generator=g) for _ in range(4))
    boost = torch.rand(b, h, t, 1, device=cuda, generator=g) < 0.1
    k = torch.where(boost, 2.0 * k, k)
    r = lambda x: x.reshape(b * h, 1, t, d)
    qq, kk, vv = (r(x).bfloat16() for x in (q, k, v))
    dd = r(do)
    del q, k, v, do, boost
    full, aux = kernels.selective_attention_forward(qq, kk, vv, return_aux=True)
    totals = aux["selected_total"]
    del aux
    part = kernels.selective_attention_forward(qq[:, :, :2048].contiguous(), kk[:, :, :2048].contiguous(),
                                               vv[:, :, :2048].contiguous())
    assert torch.equal(full[:, :, :2048], part)
    picks = (0, b * h - 1)
    oracle_totals = {}
    for sq in picks:
        sl = slice(sq, sq + 1)
        rows, want, total = sa_oracle.tail(qq[sl].double(), kk[sl].double(), vv[sl].double(), 64, chunk=4096)
        err = (full[sl][:, :, rows].double() - want).abs().max().item()
        trel = ((totals[sl].double() - total).abs().max() / total.abs().max()).item()
        print(f"C5 sequence {sq}: tail max-abs {err:.2e}, totals rel {trel:.2e}", flush=True)
        assert err < 2e-2
        assert trel < 1e-3
        oracle_totals[sq] = total
    qs, ks, vs = (x.clone().requires_grad_(True) for x in (qq, kk, vv))
    out = kernels.selective_attention(qs, ks, vs)
    assert torch.equal(out.detach(), full)
    del full, part
    dq, dk, dv = torch.autograd.grad(out, (qs, ks, vs), dd)
    for x in (dq, dk, dv):
        assert x.dtype == torch.bfloat16 and torch.isfinite(x).all()
    for sq in picks:
        sl = slice(sq, sq + 1)
        want_dv = _last_key_dv(qq[sl].double(), kk[sl].double(), dd[sl], oracle_totals[sq])
        got_dv = dv[sl][:, :, -1:].double()
        rel = ((got_dv - want_dv).abs().max() / want_dv.abs().max()).item()
        print(f"C5 sequence {sq}: last-key dV rel {rel:.2e}", flush=True)
        assert rel < 2e-2


@pytest.mark.parametrize("geometry,params", [("d768", 208_540_416), ("d1024", 353_502_208)])
def test_c3_training_step_16384(cuda, geometry, params):
    """C3: one full training step (forward, backward, clipping, fused AdamW) of the 24-layer
    decoder on 1 x 16,384 tokens under bf16 autocast, at the reference's d768 / 12-head model and
    BASELINE's d1024 / 16-head geometry: the loss and every gradient are finite, over two steps."""
    print(f"case C3 train step {geometry} T=16384", flush=True)
    cfg = ModelConfig(n_layers=24, context_length=16384, **harness.GEOMETRIES[geometry])
    torch.manual_seed(0)
    model = SelectiveLM(cfg).to(cuda).train()
    assert model.num_parameters() == params
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
