"""GPU parity of the HIP kernels (through the C ABI, via selective_attention.kernels) against the CPU
oracle, following the reference's kernel tests (reference tests/test_selective_kernels.py).

The oracle runs in float64 on the CPU on the same (operand-rounded) inputs. Tolerances:
  fp32 operands ("ieee"/"tf32", fp32 MFMA): outputs atol/rtol 2e-5, gradients atol 5e-5 rtol 5e-4
  bf16 operands: max-abs 2e-2 on out, dq, dk, dv at the C2 slice (B=1, H=16, T=2048, D=64); the
  reference's own bf16 test bounds (out max-abs 3e-2, gradient relative norm 3e-2) elsewhere.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import sa_oracle
from selective_attention import kernels

pytestmark = pytest.mark.gpu


def _qkv(batch, heads, seq, head_dim, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return tuple(scale * torch.randn(batch, heads, seq, head_dim, generator=g) for _ in range(3))


def _oracle_fwd_bwd(q, k, v, weight=None, exempt=1):
    qq, kk, vv = (t.double().requires_grad_(True) for t in (q, k, v))
    out = sa_oracle.attention(qq, kk, vv, exempt)
    if weight is None:
        return out.detach(), None
    (out * weight.double()).sum().backward()
    return out.detach(), (qq.grad, kk.grad, vv.grad)


def _kernel_fwd_bwd(q, k, v, dev, weight=None, dtype=torch.float32, **kw):
    qq, kk, vv = (t.to(dev, dtype).requires_grad_(weight is not None) for t in (q, k, v))
    out = kernels.selective_attention(qq, kk, vv, **kw)
    if weight is None:
        return out.detach().cpu(), None
    (out * weight.to(dev)).sum().backward()
    return out.detach().cpu(), (qq.grad.cpu(), kk.grad.cpu(), vv.grad.cpu())


def _close(got, want, atol, rtol, name=""):
    torch.testing.assert_close(got.double(), want.double(), atol=atol, rtol=rtol, msg=lambda m: f"{name}: {m}")


@pytest.mark.parametrize("seq", [1, 2, 31, 32, 33, 64, 65, 130, 257, 513])
@pytest.mark.parametrize("heads", [1, 3])
def test_forward_matches_oracle(cuda, seq, heads):
    print(f"case forward seq={seq} heads={heads}", flush=True)
    q, k, v = _qkv(2, heads, seq, 32, seed=seq, scale=1.5)
    got, aux = kernels.selective_attention_forward(q.to(cuda), k.to(cuda), v.to(cuda), dot_precision="ieee",
                                                   return_aux=True)
    want = sa_oracle.attention(q.double(), k.double(), v.double())
    _close(got.cpu(), want, 2e-5, 2e-5, "out")
    _close(aux["selected_total"].cpu(), sa_oracle.selection_totals(q.double(), k.double()), 2e-4, 2e-5, "total")


@pytest.mark.parametrize("head_dim", [16, 32, 64, 128])
@pytest.mark.parametrize("heads", [1, 2, 4])
def test_forward_head_dims(cuda, head_dim, heads):
    print(f"case forward head_dim={head_dim} heads={heads}", flush=True)
    q, k, v = _qkv(1, heads, 300, head_dim, seed=head_dim, scale=1.5)
    got = kernels.selective_attention_forward(q.to(cuda), k.to(cuda), v.to(cuda), dot_precision="ieee")
    _close(got.cpu(), sa_oracle.attention(q.double(), k.double(), v.double()), 2e-5, 2e-5, "out")


@pytest.mark.parametrize("head_dim", [32, 64, 128])
@pytest.mark.parametrize("blocks", [(32, 32), (64, 32), (128, 64), (None, 128)])
def test_forward_block_shapes(cuda, head_dim, blocks):
    """The reference's launch-policy arguments (block_m, block_n, num_stages; reference
    tests/test_selective_kernels.py:100-105) are accepted and validated; the HIP kernels tile by
    their own policy, so every choice returns the oracle's outputs."""
    print(f"case forward blocks={blocks} head_dim={head_dim}", flush=True)
    q, k, v = _qkv(1, 2, 300, head_dim, seed=head_dim, scale=1.5)
    got = kernels.selective_attention_forward(q.to(cuda), k.to(cuda), v.to(cuda), dot_precision="ieee",
                                              block_m=blocks[0], block_n=blocks[1], num_stages=1)
    _close(got.cpu(), sa_oracle.attention(q.double(), k.double(), v.double()), 2e-5, 2e-5, "out")


@pytest.mark.parametrize("seq", [1, 2, 33, 64, 65, 200, 513])
@pytest.mark.parametrize("heads", [1, 4])
def test_backward_matches_oracle(cuda, seq, heads):
    print(f"case backward seq={seq} heads={heads}", flush=True)
    q, k, v = _qkv(2, heads, seq, 32, seed=seq + 7, scale=1.5)
    w = torch.randn(2, heads, seq, 32, generator=torch.Generator().manual_seed(seq))
    out, grads = _kernel_fwd_bwd(q, k, v, cuda, w, dot_precision="ieee")
    want, wgrads = _oracle_fwd_bwd(q, k, v, w)
    _close(out, want, 5e-5, 5e-4, "out")
    for name, g, wg in zip(("dq", "dk", "dv"), grads, wgrads):
        _close(g, wg, 5e-5, 5e-4, name)


@pytest.mark.parametrize("head_dim", [16, 64, 128])
def test_backward_head_dims(cuda, head_dim):
    print(f"case backward head_dim={head_dim}", flush=True)
    q, k, v = _qkv(1, 4, 150, head_dim, seed=head_dim + 1, scale=1.5)
    w = torch.randn(1, 4, 150, head_dim, generator=torch.Generator().manual_seed(3))
    out, grads = _kernel_fwd_bwd(q, k, v, cuda, w, dot_precision="ieee")
    want, wgrads = _oracle_fwd_bwd(q, k, v, w)
    for name, g, wg in zip(("dq", "dk", "dv"), grads, wgrads):
        _close(g, wg, 5e-5, 5e-4, name)


def test_selection_gradient_reaches_head_zero_only_through_the_history_term(cuda):
    """Loss on heads >= 1 still reaches head 0's q and k through F, and not head 0's v
    (reference tests/test_selective_kernels.py:88-100)."""
    q, k, v = _qkv(1, 3, 97, 32, seed=3, scale=2.0)
    qq, kk, vv = (t.to(cuda).requires_grad_(True) for t in (q, k, v))
    kernels.selective_attention(qq, kk, vv, dot_precision="ieee")[:, 1:].sum().backward()
    rq, rk, rv = (t.double().requires_grad_(True) for t in (q, k, v))
    sa_oracle.attention(rq, rk, rv)[:, 1:].sum().backward()
    assert rq.grad[:, 0].abs().max() > 1e-4 and rv.grad[:, 0].abs().max() == 0
    assert vv.grad[:, 0].abs().max().item() == 0.0
    for got, want, name in ((qq.grad, rq.grad, "dq"), (kk.grad, rk.grad, "dk"), (vv.grad, rv.grad, "dv")):
        _close(got.cpu(), want, 5e-5, 5e-4, name)


@pytest.mark.parametrize("heads,group,bwd_group", [(2, 2, 2), (4, 4, 2), (6, 2, 1), (12, 4, 2), (12, 4, 1),
                                                   (5, None, None), (8, 1, 1)])
@pytest.mark.parametrize("seq", [1, 33, 257])
def test_grouped_launches_match_oracle(cuda, heads, group, bwd_group, seq):
    print(f"case grouped heads={heads} group={group} bwd_group={bwd_group} seq={seq}", flush=True)
    q, k, v = _qkv(2, heads, seq, 32, seed=seq + heads, scale=1.5)
    w = torch.randn(2, heads, seq, 32, generator=torch.Generator().manual_seed(seq))
    out, grads = _kernel_fwd_bwd(q, k, v, cuda, w, dot_precision="ieee", group=group, bwd_group=bwd_group)
    want, wgrads = _oracle_fwd_bwd(q, k, v, w)
    _close(out, want, 5e-5, 5e-4, "out")
    for name, g, wg in zip(("dq", "dk", "dv"), grads, wgrads):
        _close(g, wg, 5e-5, 5e-4, name)


@pytest.mark.parametrize("heads,group", [(4, 1), (4, 2), (4, 4), (8, 4)])
def test_bf16_grouped_launches_match_oracle(cuda, heads, group):
    """bf16 operands, every forward head-group width the kernels instantiate."""
    print(f"case bf16 grouped heads={heads} group={group}", flush=True)
    q, k, v = (t.bfloat16() for t in _qkv(1, heads, 257, 64, seed=heads + group))
    w = torch.randn(1, heads, 257, 64, generator=torch.Generator().manual_seed(5))
    out, grads = _kernel_fwd_bwd(q, k, v, cuda, w, dtype=torch.bfloat16, group=group)
    want, wgrads = _oracle_fwd_bwd(q, k, v, w)
    assert (out.double() - want).abs().max() < 3e-2
    for g, wg in zip(grads, wgrads):
        assert ((g.double() - wg).norm() / wg.norm()) < 3e-2


@pytest.mark.parametrize("precision", ["bf16", "tf32"])
def test_low_precision_paths_stay_close(cuda, precision):
    """reference tests/test_selective_kernels.py:103-119"""
    q, k, v = _qkv(2, 4, 400, 64, seed=11)
    dtype = torch.float32
    if precision == "bf16":
        q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
        dtype = torch.bfloat16
    qq, kk, vv = (t.to(cuda).requires_grad_(True) for t in (q, k, v))
    got = kernels.selective_attention(qq, kk, vv, dot_precision=precision)
    want = sa_oracle.attention(q.double(), k.double(), v.double())
    assert (got.detach().cpu().double() - want).abs().max() < 3e-2
    got.float().pow(2).sum().backward()
    rq, rk, rv = (t.double().requires_grad_(True) for t in (q, k, v))
    sa_oracle.attention(rq, rk, rv).pow(2).sum().backward()
    for g, wg in ((qq.grad, rq.grad), (kk.grad, rk.grad), (vv.grad, rv.grad)):
        assert g.dtype == dtype
        err = (g.cpu().double() - wg).norm() / wg.norm()
        assert err < 3e-2, float(err)


def test_long_sequence_forward_and_backward(cuda):
    """Many carry checkpoints, a partial last tile (reference tests/test_selective_kernels.py:122-136)."""
    q, k, v = _qkv(1, 2, 2049, 32, seed=5, scale=1.2)
    w = torch.randn(1, 2, 2049, 32, generator=torch.Generator().manual_seed(9))
    out, grads = _kernel_fwd_bwd(q, k, v, cuda, w, dot_precision="ieee")
    want, wgrads = _oracle_fwd_bwd(q, k, v, w)
    _close(out, want, 5e-5, 5e-5, "out")
    for g, wg in zip(grads, wgrads):
        assert ((g.double() - wg).norm() / wg.norm()) < 1e-3


@pytest.mark.parametrize("exempt", [1, 3, 16, 40])
@pytest.mark.parametrize("group", [1, None])
def test_exempt_matches_oracle(cuda, exempt, group):
    q, k, v = _qkv(2, 4, 257, 32, seed=exempt, scale=1.5)
    w = torch.randn(2, 4, 257, 32, generator=torch.Generator().manual_seed(exempt))
    out, grads = _kernel_fwd_bwd(q, k, v, cuda, w, dot_precision="ieee", group=group, bwd_group=group,
                                 exempt=exempt)
    want, wgrads = _oracle_fwd_bwd(q, k, v, w, exempt=exempt)
    _close(out, want, 5e-5, 5e-4, "out")
    for name, g, wg in zip(("dq", "dk", "dv"), grads, wgrads):
        _close(g, wg, 5e-5, 5e-4, name)
    _, aux = kernels.selective_attention_forward(q.to(cuda), k.to(cuda), v.to(cuda), dot_precision="ieee",
                                                 return_aux=True, exempt=exempt)
    _close(aux["selected_total"].cpu(), sa_oracle.selection_totals(q.double(), k.double(), exempt), 2e-4, 2e-5,
           "total")


@pytest.mark.parametrize("damp", ["linear", "sqrt"])
@pytest.mark.parametrize("heads,group", [(3, 1), (4, 4), (4, 2)])
def test_history_damping(cuda, damp, heads, group):
    """reference tests/test_selective_kernels.py:223-242"""
    q, k, v = _qkv(1, heads, 300, 32, seed=17, scale=1.5)
    qd, kd, vd = (t.to(cuda) for t in (q, k, v))
    plain = kernels.selective_attention_forward(qd, kd, vd, dot_precision="ieee", group=group)
    inside = kernels.selective_attention_forward(qd, kd, vd, dot_precision="ieee", group=group, damp=damp,
                                                 train_len=300)
    torch.testing.assert_close(inside, plain)
    got = kernels.selective_attention_forward(qd, kd, vd, dot_precision="ieee", group=group, damp=damp,
                                              train_len=100)
    qq, kk, vv = q.double(), k.double(), v.double()
    raw = sa_oracle.raw_logits(qq, kk)
    hist = sa_oracle.history(sa_oracle.selection(qq, kk))[:, None]
    scale = (100.0 / torch.arange(1, 301, dtype=torch.float64)).clamp(max=1.0)
    if damp == "sqrt":
        scale = scale.sqrt()
    lg = (raw - hist * scale[:, None]).masked_fill(~torch.ones(300, 300, dtype=torch.bool).tril(), float("-inf"))
    _close(got.cpu(), lg.softmax(-1) @ vv, 2e-5, 2e-5, "damped out")


def test_default_precision_follows_the_input_dtype(cuda):
    q, k, v = (t.to(cuda) for t in _qkv(1, 4, 200, 32, seed=8))
    torch.testing.assert_close(kernels.selective_attention_forward(q, k, v),
                               kernels.selective_attention_forward(q, k, v, dot_precision="tf32"))
    qb, kb, vb = q.bfloat16(), k.bfloat16(), v.bfloat16()
    torch.testing.assert_close(kernels.selective_attention_forward(qb, kb, vb),
                               kernels.selective_attention_forward(qb, kb, vb, dot_precision="bf16"))
    torch.testing.assert_close(kernels.selective_attention(qb, kb, vb),
                               kernels.selective_attention(qb, kb, vb, dot_precision="bf16"))


def test_fp16_inputs(cuda):
    q, k, v = (t.half() for t in _qkv(1, 2, 100, 64, seed=4))
    qq, kk, vv = (t.to(cuda).requires_grad_(True) for t in (q, k, v))
    out = kernels.selective_attention(qq, kk, vv)
    want = sa_oracle.attention(q.double(), k.double(), v.double())
    _close(out.detach().cpu(), want, 1e-4, 1e-4, "fp16 via fp32 operands")
    out.sum().backward()
    assert qq.grad.dtype == torch.float16 and torch.isfinite(qq.grad).all()


def test_bad_inputs_raise_clear_errors(cuda):
    q, k, v = (t.to(cuda) for t in _qkv(1, 2, 64, 32))
    with pytest.raises(ValueError, match="must all be"):
        kernels.selective_attention(q, k[:, :, :32], v)
    with pytest.raises(ValueError, match="CUDA"):
        kernels.selective_attention(q.cpu(), k.cpu(), v.cpu())
    with pytest.raises(ValueError, match="dtype"):
        kernels.selective_attention(q.double(), k.double(), v.double())
    with pytest.raises(ValueError, match="head_dim"):
        kernels.selective_attention(q[..., :24], k[..., :24], v[..., :24])
    with pytest.raises(ValueError, match="dot_precision"):
        kernels.selective_attention(q, k, v, dot_precision="fp8")
    with pytest.raises(ValueError, match="exempt"):
        kernels.selective_attention(q, k, v, exempt=0)
    with pytest.raises(ValueError, match="bwd_group"):
        kernels.selective_attention(q.requires_grad_(True), k, v, bwd_group=4).sum().backward()
    with pytest.raises(ValueError, match="damp"):
        kernels.selective_attention_forward(q, k, v, damp="cubic", train_len=10)
    with pytest.raises(TypeError):
        kernels.selective_attention_forward(q, k, v, None, None, 32, False, 4, None, None, 1, "linear")
    assert kernels.supported(q) and not kernels.supported(q.cpu()) and not kernels.supported(q[..., :24])


# -- chunked prefill and per-head selection ---------------------------------------------------------

@pytest.mark.parametrize("seq,chunk", [(300, 64), (257, 100), (96, 32), (70, 1)])
def test_chunked_prefill_equals_single_shot(cuda, seq, chunk):
    print(f"case prefill seq={seq} chunk={chunk}", flush=True)
    q, k, v = _qkv(2, 3, seq, 32, seed=seq + chunk, scale=1.5)
    qd, kd, vd = (t.to(cuda) for t in (q, k, v))
    state = torch.zeros(2, seq, device=cuda)
    outs = []
    for c0 in range(0, seq, chunk):
        c1 = min(seq, c0 + chunk)
        outs.append(kernels.selective_attention_prefill(qd[:, :, c0:c1], kd[:, :, :c1], vd[:, :, :c1], state, c0,
                                                        dot_precision="ieee"))
    got = torch.cat(outs, dim=2).cpu()
    want, want_state = sa_oracle.prefill_chunks(q.double(), k.double(), v.double(), chunk)
    _close(got, sa_oracle.attention(q.double(), k.double(), v.double()), 2e-5, 2e-5, "chunked out")
    _close(state.cpu(), want_state, 2e-4, 2e-5, "state")


def test_chunked_prefill_bf16_matches_single_shot_kernel(cuda):
    q, k, v = (t.bfloat16().to(cuda) for t in _qkv(1, 4, 1024, 64, seed=21))
    full = kernels.selective_attention_forward(q, k, v)
    state = torch.zeros(1, 1024, device=cuda)
    outs = [kernels.selective_attention_prefill(q[:, :, c0:c0 + 256], k[:, :, :c0 + 256], v[:, :, :c0 + 256], state, c0)
            for c0 in range(0, 1024, 256)]
    got = torch.cat(outs, dim=2)
    assert (got - full).abs().max().item() < 1e-2


def test_per_head_selection_matches_each_head_alone(cuda):
    """reference tests/test_selective_perhead.py:25-29: per-head mode is each head as its own
    one-head sequence."""
    q, k, v = _qkv(2, 4, 130, 32, seed=2, scale=1.5)
    w = torch.randn(2, 4, 130, 32, generator=torch.Generator().manual_seed(2))
    r = lambda t: t.reshape(8, 1, 130, 32)
    out, grads = _kernel_fwd_bwd(r(q), r(k), r(v), cuda, r(w), dot_precision="ieee")
    qq, kk, vv = (t.double().requires_grad_(True) for t in (q, k, v))
    want = sa_oracle.per_head(qq, kk, vv)
    (want * w.double()).sum().backward()
    _close(out.reshape(2, 4, 130, 32), want.detach(), 5e-5, 5e-4, "out")
    for name, g, wg in zip(("dq", "dk", "dv"), grads, (qq.grad, kk.grad, vv.grad)):
        _close(g.reshape(2, 4, 130, 32), wg, 5e-5, 5e-4, name)


# -- BASELINE configurations ---------------------------------------------------------------------------

def _c2_slice_inputs():
    g = torch.Generator().manual_seed(1234)
    return tuple(torch.randn(1, 16, 2048, 64, generator=g).bfloat16() for _ in range(4))


def test_c2_slice_bf16_within_2e_2(cuda):
    """C2 parity: bf16-operand fwd+bwd at B=1, H=16, T=2048, D=64 against the fp64 oracle on the same
    bf16-valued inputs; max-abs 2e-2 on out, dq, dk, dv. The inputs are fp32 tensors holding bf16
    values with dot_precision="bf16": the kernels run exactly the bf16 MFMA path and return the fp32
    gradient accumulators (gradients follow the input dtype, as in the reference)."""
    q, k, v, do = _c2_slice_inputs()
    qq, kk, vv = (t.float().to(cuda).requires_grad_(True) for t in (q, k, v))
    out = kernels.selective_attention(qq, kk, vv, dot_precision="bf16")
    out.backward(do.to(cuda).float())
    assert qq.grad.dtype == torch.float32
    want, wgrads = _oracle_fwd_bwd(q, k, v, do.float())
    errs = {"out": (out.detach().cpu().double() - want).abs().max().item()}
    for name, gr, wg in zip(("dq", "dk", "dv"), (qq.grad, kk.grad, vv.grad), wgrads):
        errs[name] = (gr.cpu().double() - wg).abs().max().item()
    print("C2 slice max-abs errors:", errs, flush=True)
    assert all(e < 2e-2 for e in errs.values()), errs


def test_c2_slice_bf16_inputs_bf16_gradients(cuda):
    """The same slice with bf16 tensors: gradients come back in bf16, so each element also carries
    the rounding of its own bf16 representation (half an ulp: up to 0.0625 at |g| in [16, 32))."""
    q, k, v, do = _c2_slice_inputs()
    qq, kk, vv = (t.to(cuda).requires_grad_(True) for t in (q, k, v))
    out = kernels.selective_attention(qq, kk, vv)
    out.backward(do.to(cuda).float())
    want, wgrads = _oracle_fwd_bwd(q, k, v, do.float())
    assert (out.detach().cpu().double() - want).abs().max().item() < 2e-2
    for name, gr, wg in zip(("dq", "dk", "dv"), (qq.grad, kk.grad, vv.grad), wgrads):
        assert gr.dtype == torch.bfloat16
        wb = wg.to(torch.bfloat16).double()
        half_ulp = (wb.abs() * 2.0 ** -8).clamp(min=2.0 ** -133)
        excess = ((gr.cpu().double() - wg).abs() - half_ulp).max().item()
        assert excess < 2e-2, (name, excess)


def test_c2_full_length_prefix_is_exact(cuda):
    """At T=16384 (C2's length) the first 2048 rows equal the T=2048 run bit for bit (causality), the
    last rows and the selection totals agree with the oracle's chunk-summed tail form, and the full
    backward at that length returns finite gradients in the inputs' dtype."""
    g = torch.Generator().manual_seed(77)
    q, k, v = (torch.randn(1, 16, 16384, 64, generator=g).bfloat16().to(cuda) for _ in range(3))
    full, aux = kernels.selective_attention_forward(q, k, v, return_aux=True)
    part = kernels.selective_attention_forward(q[:, :, :2048].contiguous(), k[:, :, :2048].contiguous(),
                                               v[:, :, :2048].contiguous())
    assert torch.equal(full[:, :, :2048], part)
    rows, want, total = sa_oracle.tail(q.cpu().float(), k.cpu().float(), v.cpu().float(), 64, chunk=2048)
    got = full[:, :, rows].cpu()
    assert (got - want).abs().max().item() < 2e-2
    rel = (aux["selected_total"].cpu() - total).abs().max() / total.abs().max()
    assert rel.item() < 1e-2
    qq, kk, vv = (t.requires_grad_(True) for t in (q, k, v))
    out = kernels.selective_attention(qq, kk, vv)
    torch.testing.assert_close(out.detach(), full, rtol=0, atol=0)
    out.backward(torch.randn(out.shape, device=cuda, generator=torch.Generator(device=cuda).manual_seed(5)))
    for t in (qq, kk, vv):
        assert t.grad.dtype == torch.bfloat16 and torch.isfinite(t.grad).all()


def test_c1_fp32_forward_within_1e_4_relative(cuda):
    """C1: B=1, H=4, T=512, D=64, fp32, q, k, v ~ N(0,1) from one seed drawn in q, k, v order; the
    fp32 kernel path (dot_precision="ieee") against the oracle, within 1e-4 relative
    (||delta||_inf / ||ref||_inf)."""
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, 4, 512, 64, generator=g) for _ in range(3))
    got = kernels.selective_attention_forward(q.to(cuda), k.to(cuda), v.to(cuda), dot_precision="ieee")
    want = sa_oracle.attention(q.double(), k.double(), v.double())
    rel = (got.cpu().double() - want).abs().max() / want.abs().max()
    assert rel.item() < 1e-4, rel.item()
    # and the fp32 listing in the reference's own form (kernels.selective_attention_reference)
    lst = kernels.selective_attention_reference(q, k, v)
    assert ((lst.double() - want).abs().max() / want.abs().max()).item() < 1e-5


def test_c5_per_head_slice_bf16_within_2e_2(cuda):
    """C5 parity on a T=2048 slice: per-head selection (every head its own selector), bf16 operands,
    k scaled by 2 on a random 10% of key positions; out, dq, dk, dv within 2e-2 max-abs against the
    per-head oracle (fp32 tensors holding bf16 values, so the gradients stay fp32)."""
    g = torch.Generator().manual_seed(55)
    b, h, t, d = 2, 16, 2048, 64
    q, k, v, do = (torch.randn(b, h, t, d, generator=g) for _ in range(4))
    boost = torch.rand(b, h, t, 1, generator=g) < 0.1
    k = torch.where(boost, 2.0 * k, k)
    q, k, v, do = (x.bfloat16().float() for x in (q, k, v, do))
    r = lambda x: x.reshape(b * h, 1, t, d)
    qq, kk, vv = (r(x).to(cuda).requires_grad_(True) for x in (q, k, v))
    out = kernels.selective_attention(qq, kk, vv, dot_precision="bf16")
    out.backward(r(do).to(cuda))
    errs = {}
    for hh in range(0, b * h, 8):   # the oracle on every sequence (each one head), 8 at a time
        sl = slice(hh, hh + 8)
        rq, rk, rv = (x[sl].double().requires_grad_(True) for x in (r(q), r(k), r(v)))
        ref = sa_oracle.attention(rq, rk, rv)
        ref.backward(r(do)[sl].double())
        for name, got, want in (("out", out.detach()[sl], ref.detach()), ("dq", qq.grad[sl], rq.grad),
                                ("dk", kk.grad[sl], rk.grad), ("dv", vv.grad[sl], rv.grad)):
            errs[name] = max(errs.get(name, 0.0), (got.cpu().double() - want).abs().max().item())
    print("C5 slice max-abs errors:", errs, flush=True)
    assert all(e < 2e-2 for e in errs.values()), errs


@pytest.mark.parametrize("chunk", [7, 13, 33])
@pytest.mark.parametrize("exempt", [1, 16])
def test_chunked_prefill_unaligned_offsets(cuda, chunk, exempt):
    """Chunk offsets that are not multiples of the 32-query tile: the key tile ending at a chunk's
    first query must still exclude that query's own key from its selection."""
    print(f"case prefill unaligned chunk={chunk} exempt={exempt}", flush=True)
    q, k, v = _qkv(2, 4, 160, 32, seed=chunk + exempt, scale=1.5)
    qd, kd, vd = (t.to(cuda) for t in (q, k, v))
    state = torch.zeros(2, 160, device=cuda)
    outs = [kernels.selective_attention_prefill(qd[:, :, c0:c0 + chunk], kd[:, :, :c0 + chunk], vd[:, :, :c0 + chunk],
                                                state, c0, dot_precision="ieee", exempt=exempt)
            for c0 in range(0, 160, chunk)]
    want = sa_oracle.attention(q.double(), k.double(), v.double(), exempt)
    _close(torch.cat(outs, dim=2).cpu(), want, 2e-5, 2e-5, "chunked out")
    _close(state.cpu(), sa_oracle.selection_totals(q.double(), k.double(), exempt), 2e-4, 2e-5, "state")
