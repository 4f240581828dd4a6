"""bf16-operand parity of every kernel instance the library ships, against the fp64 oracle on the same
bf16-valued inputs (reference tests/test_selective_kernels.py:141-172, 203-242).

The launch policy picks the instance from (head_dim, heads, group, bwd_group); with H = 4:

    forward   head_dim 16 / 32 (run at 32): group 1 -> 1 head per wavefront, 2 -> 2, 4 / None -> 4
              head_dim 64:                  group 1 -> 1, 2 -> 2, 4 -> 4, None -> 2, or 1 when
                                            the two-head grid fills the CUs only once (the same bits:
                                            test_fwd64_one_or_two_heads_per_wavefront_same_bits; an
                                            odd head count runs 1: the prefill cases at H = 3 and 1)
              head_dim 128:                 1
    backward  head_dim 16 / 32: bwd_group 2 -> 2 heads per wavefront (key side and query side),
              1 / None -> 1;  head_dim 64, 128: 1

so the parameter grid below runs each forward width at head dims 32 and 64, the two-head backward at
32, and both storage layouts (split heads: contiguous instances; packed projection: view instances).
Bounds are the reference's bf16 bounds: output max-abs 3e-2, gradient relative norm 3e-2.
"""

from __future__ import annotations

import pytest
import torch

from oracle import sa_oracle
from selective_attention import kernels

pytestmark = pytest.mark.gpu


def _inputs(batch, heads, seq, head_dim, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    q, k, v, w = (torch.randn(batch, heads, seq, head_dim, generator=g) for _ in range(4))
    return (scale * q).bfloat16(), (scale * k).bfloat16(), (scale * v).bfloat16(), w


def _oracle(q, k, v, w, exempt=1):
    qq, kk, vv = (t.double().requires_grad_(True) for t in (q, k, v))
    out = sa_oracle.attention(qq, kk, vv, exempt)
    (out * w.double()).sum().backward()
    return out.detach(), (qq.grad, kk.grad, vv.grad)


def _kernel(q, k, v, w, dev, **kw):
    qq, kk, vv = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    out = kernels.selective_attention(qq, kk, vv, **kw)
    (out * w.to(dev)).sum().backward()
    return out.detach().cpu(), tuple(t.grad.cpu() for t in (qq, kk, vv))


def _check(out, grads, want, wgrads, tag):
    err = (out.double() - want).abs().max().item()
    rel = [((g.double() - wg).norm() / wg.norm()).item() for g, wg in zip(grads, wgrads)]
    print(f"{tag}: out max-abs {err:.2e}, grad rel-norm {rel}", flush=True)
    assert err < 3e-2, (tag, err)
    assert all(r < 3e-2 for r in rel), (tag, rel)


@pytest.mark.parametrize("head_dim", [16, 32, 64, 128])
@pytest.mark.parametrize("group,bwd_group", [(1, 1), (2, 2), (4, None), (None, None)])
def test_bf16_instances_match_oracle(cuda, head_dim, group, bwd_group):
    tag = f"bf16 D={head_dim} group={group} bwd_group={bwd_group}"
    print("case", tag, flush=True)
    q, k, v, w = _inputs(2, 4, 257, head_dim, seed=head_dim + 10 * (group or 0) + (bwd_group or 0))
    out, grads = _kernel(q, k, v, w, cuda, group=group, bwd_group=bwd_group)
    assert all(g.dtype == torch.bfloat16 for g in grads)
    _check(out, grads, *_oracle(q, k, v, w), tag)


@pytest.mark.parametrize("head_dim,heads,exempt", [(32, 4, 3), (32, 4, 40), (64, 4, 16), (64, 2, 3),
                                                   (128, 2, 40)])
def test_bf16_exempt_matches_oracle(cuda, head_dim, heads, exempt):
    """Wide exempt prefixes on the bf16 instances (reference tests/test_selective_kernels.py:203-220):
    keys below `exempt` are never selected and take the split-operand products."""
    tag = f"bf16 exempt={exempt} D={head_dim} H={heads}"
    print("case", tag, flush=True)
    q, k, v, w = _inputs(1, heads, 300, head_dim, seed=exempt + head_dim, scale=1.3)
    out, grads = _kernel(q, k, v, w, cuda, exempt=exempt, bwd_group=2)
    _check(out, grads, *_oracle(q, k, v, w, exempt), tag)
    _, aux = kernels.selective_attention_forward(q.to(cuda), k.to(cuda), v.to(cuda), return_aux=True,
                                                 exempt=exempt)
    want = sa_oracle.selection_totals(q.double(), k.double(), exempt)
    got = aux["selected_total"].cpu().double()
    assert ((got - want).abs().max() / want.abs().max()).item() < 1e-4


@pytest.mark.parametrize("damp", ["linear", "sqrt"])
@pytest.mark.parametrize("head_dim,group", [(32, 4), (32, 2), (64, None), (64, 1), (128, None)])
def test_bf16_history_damping(cuda, damp, head_dim, group):
    """Evaluation-only history damping on the bf16 forward instances (reference
    tests/test_selective_kernels.py:223-242): damping with train_len >= T changes nothing, and with
    train_len < T the forward equals the listing with query i's history scaled by
    min(1, train_len / (i + 1)) (or its square root)."""
    print(f"case bf16 damping {damp} D={head_dim} group={group}", flush=True)
    q, k, v, _ = _inputs(1, 4, 300, head_dim, seed=17, scale=1.3)
    qd, kd, vd = (t.to(cuda) for t in (q, k, v))
    plain = kernels.selective_attention_forward(qd, kd, vd, group=group)
    inside = kernels.selective_attention_forward(qd, kd, vd, group=group, damp=damp, train_len=300)
    torch.testing.assert_close(inside, plain, rtol=0, atol=0)
    got = kernels.selective_attention_forward(qd, kd, vd, group=group, damp=damp, train_len=100)
    qq, kk, vv = q.double(), k.double(), v.double()
    raw = sa_oracle.raw_logits(qq, kk)
    hist = sa_oracle.history(sa_oracle.selection(qq, kk))[:, None]
    scale = (100.0 / torch.arange(1, 301, dtype=torch.float64)).clamp(max=1.0)
    if damp == "sqrt":
        scale = scale.sqrt()
    lg = (raw - hist * scale[:, None]).masked_fill(~torch.ones(300, 300, dtype=torch.bool).tril(), float("-inf"))
    err = (got.cpu().double() - lg.softmax(-1) @ vv).abs().max().item()
    assert err < 3e-2, err
    # the damping must matter at these inputs (else the check above would not test it)
    assert (got - plain).abs().max().item() > 0.1


@pytest.mark.parametrize("head_dim,heads,chunk", [(64, 4, 256), (64, 3, 300), (64, 1, 192), (32, 4, 100),
                                                  (128, 2, 333)])
def test_bf16_chunked_prefill_matches_oracle(cuda, head_dim, heads, chunk):
    """Chunked prefill on the bf16 instances against the oracle (output and carried state), and
    against the single-shot bf16 forward."""
    print(f"case bf16 prefill D={head_dim} H={heads} chunk={chunk}", flush=True)
    t = 1000
    q, k, v, _ = _inputs(1, heads, t, head_dim, seed=chunk + head_dim)
    qd, kd, vd = (x.to(cuda) for x in (q, k, v))
    state = torch.zeros(1, t, device=cuda)
    outs = [kernels.selective_attention_prefill(qd[:, :, c0:c0 + chunk], kd[:, :, :c0 + chunk],
                                                vd[:, :, :c0 + chunk], state, c0)
            for c0 in range(0, t, chunk)]
    got = torch.cat(outs, dim=2)
    want = sa_oracle.attention(q.double(), k.double(), v.double())
    assert (got.cpu().double() - want).abs().max().item() < 3e-2
    total = sa_oracle.selection_totals(q.double(), k.double())
    assert ((state.cpu().double() - total).abs().max() / total.abs().max()).item() < 1e-4
    full = kernels.selective_attention_forward(qd, kd, vd)
    assert (got - full).abs().max().item() < 1e-2


@pytest.mark.parametrize("head_dim,heads", [(32, 4), (64, 4), (128, 2)])
def test_bf16_packed_projection_matches_oracle(cuda, head_dim, heads):
    """The view instances (q, k, v read in place from a packed (B, T, 3 * H * D) projection; gradient
    written as one packed tensor) against the oracle."""
    print(f"case bf16 packed D={head_dim} H={heads}", flush=True)
    g = torch.Generator().manual_seed(head_dim)
    b, t = 2, 230
    qkv = torch.randn(b, t, 3 * heads * head_dim, generator=g).bfloat16()
    dy = torch.randn(b, t, heads * head_dim, generator=g)
    x = qkv.to(cuda).requires_grad_(True)
    y = kernels.selective_attention_qkv(x, heads)
    y.backward(dy.bfloat16().to(cuda))
    xr = qkv.double().requires_grad_(True)
    parts = xr.view(b, t, 3, heads, head_dim)
    q, k, v = (parts[:, :, i].transpose(1, 2) for i in range(3))
    o = sa_oracle.attention(q, k, v)
    yr = o.transpose(1, 2).reshape(b, t, heads * head_dim)
    yr.backward(dy.bfloat16().double())
    assert (y.detach().cpu().double() - yr.detach()).abs().max().item() < 3e-2
    got, want = (z.view(b, t, 3, heads, head_dim) for z in (x.grad.cpu().double(), xr.grad))
    for i, name in enumerate(("dq", "dk", "dv")):
        rel = ((got[:, :, i] - want[:, :, i]).norm() / want[:, :, i].norm()).item()
        assert rel < 3e-2, (name, rel)


@pytest.mark.parametrize("seq", [1, 2, 31, 32, 33, 64, 65, 97, 160])
@pytest.mark.parametrize("heads", [1, 2, 3])
def test_bf16_head_dim_64_forward_short_sequences(cuda, seq, heads):
    """The direct-load forward at head dim 64 (two heads per wavefront at H = 2, one at H = 1, 3) on
    sequences of one to five key tiles: its selection runs one tile ahead and its loads two, so the
    first and last tiles of a workgroup take the loop's edge cases."""
    print(f"case bf16 D=64 short seq={seq} heads={heads}", flush=True)
    q, k, v, _ = _inputs(2, heads, seq, 64, seed=seq + 7 * heads, scale=1.3)
    got, aux = kernels.selective_attention_forward(q.to(cuda), k.to(cuda), v.to(cuda), return_aux=True)
    want = sa_oracle.attention(q.double(), k.double(), v.double())
    assert (got.cpu().double() - want).abs().max().item() < 3e-2
    total = sa_oracle.selection_totals(q.double(), k.double())
    err = (aux["selected_total"].cpu().double() - total).abs().max().item()
    assert err <= 1e-4 * max(total.abs().max().item(), 1.0), err


@pytest.mark.parametrize("batch,heads,seq,exempt,damp", [(1, 4, 300, 1, None), (2, 12, 2047, 1, None),
                                                         (1, 2, 4096, 16, None), (1, 16, 1024, 3, None),
                                                         (1, 6, 700, 1, "linear")])
def test_fwd64_one_or_two_heads_per_wavefront_same_bits(cuda, batch, heads, seq, exempt, damp):
    """At head dim 64 the library chooses one or two heads per wavefront per launch (group=None) from
    the size of the launch's grid; a shape's output must not depend on that choice, so that a prefix
    of a longer run (which may launch with the other width) stays equal bit for bit. Both widths, and
    the automatic choice, give the same output and selection state."""
    print(f"case fwd64 widths B={batch} H={heads} T={seq} E={exempt} damp={damp}", flush=True)
    q, k, v, _ = _inputs(batch, heads, seq, 64, seed=seq + heads, scale=1.2)
    qd, kd, vd = (t.to(cuda) for t in (q, k, v))
    kw = dict(exempt=exempt, return_aux=True)
    if damp:
        kw.update(damp=damp, train_len=seq // 3)
    runs = [kernels.selective_attention_forward(qd, kd, vd, group=g, **kw) for g in (1, 2, None)]
    for out, aux in runs[1:]:
        assert torch.equal(out, runs[0][0])
        assert torch.equal(aux["carry"], runs[0][1]["carry"])
        assert torch.equal(aux["selected_total"], runs[0][1]["selected_total"])
    if seq <= 1024 and not damp:   # and it is the oracle's
        with torch.no_grad():
            want = sa_oracle.attention(q.double(), k.double(), v.double(), exempt)
        assert (runs[0][0].cpu().double() - want).abs().max().item() < 3e-2


def test_fwd64_prefill_widths_same_bits(cuda):
    """The chunked prefill (a query offset, keys of earlier chunks, a carried per-key state) gives the
    same bits and the same state at one and two heads per wavefront and with the automatic choice
    (one head per wavefront here: each chunk's grid fills the CUs less than once)."""
    b, h, t, chunk = 2, 6, 3072, 1024
    print(f"case fwd64 prefill widths B={b} H={h} T={t} chunk={chunk}", flush=True)
    q, k, v, _ = _inputs(b, h, t, 64, seed=61, scale=1.2)
    qd, kd, vd = (x.to(cuda) for x in (q, k, v))
    runs = []
    for g in (1, 2, None):
        state = torch.zeros(b, t, device=cuda)
        outs = [kernels.selective_attention_prefill(qd[:, :, c0:c0 + chunk], kd[:, :, :c0 + chunk],
                                                    vd[:, :, :c0 + chunk], state, c0, group=g)
                for c0 in range(0, t, chunk)]
        runs.append((torch.cat(outs, dim=2), state))
    for out, state in runs[1:]:
        assert torch.equal(out, runs[0][0])
        assert torch.equal(state, runs[0][1])
