"""Pins of the CPU oracle (oracle/sa_oracle.py) against the operator's definition, closed forms and
finite differences; and the package's exported listing against the oracle. CPU only."""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import sa_oracle
from selective_attention import kernels


def _qkv(batch, heads, seq, head_dim, seed=0, scale=1.0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return tuple((scale * torch.randn(batch, heads, seq, head_dim, generator=g)).to(dtype) for _ in range(3))


def test_attention_matches_per_query_loop():
    """Matrix form vs the per-query running-vector form (reference tests/test_selective_kernels.py:24-40)."""
    q, k, v = _qkv(2, 3, 23, 16, scale=1.5)
    out_loop, total_loop = sa_oracle.attention_loop(q, k, v)
    torch.testing.assert_close(sa_oracle.attention(q, k, v), out_loop, atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(sa_oracle.selection_totals(q, k), total_loop, atol=1e-12, rtol=1e-12)


@pytest.mark.parametrize("exempt", [1, 2, 5])
def test_loop_form_with_exempt(exempt):
    q, k, v = _qkv(1, 2, 17, 8, seed=exempt, scale=2.0)
    out_loop, total_loop = sa_oracle.attention_loop(q, k, v, exempt)
    torch.testing.assert_close(sa_oracle.attention(q, k, v, exempt), out_loop, atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(sa_oracle.selection_totals(q, k, exempt), total_loop, atol=1e-12, rtol=1e-12)


def test_bos_column_and_diagonal_are_never_masked():
    """reference tests/test_selective_kernels.py:43-49"""
    q, k, _ = _qkv(1, 2, 12, 16, scale=3.0)
    logits, total = sa_oracle.adjusted_logits(q, k)
    raw = sa_oracle.raw_logits(q, k)
    torch.testing.assert_close(logits[..., 0], raw[..., 0])
    torch.testing.assert_close(logits.diagonal(dim1=-2, dim2=-1), raw.diagonal(dim1=-2, dim2=-1))
    assert total[0, 0] == 0 and total[0, -1] == 0


def test_exempt_positions_are_never_masked():
    """reference tests/test_selective_kernels.py:193-200"""
    q, k, _ = _qkv(1, 2, 20, 16, scale=3.0)
    for exempt in (1, 4):
        logits, total = sa_oracle.adjusted_logits(q, k, exempt)
        raw = sa_oracle.raw_logits(q, k).masked_fill(~torch.ones(20, 20, dtype=torch.bool).tril(), float("-inf"))
        torch.testing.assert_close(logits[..., :exempt], raw[..., :exempt])
        assert torch.all(total[..., :exempt] == 0) and float(total[..., exempt:].sum()) > 0


def test_history_vanishes_just_below_the_diagonal():
    """F[i, i-1] = 0: the only query that could select key i-1 before query i would be earlier than i-1."""
    q, k, _ = _qkv(1, 1, 30, 8, scale=2.0)
    logits, _ = sa_oracle.adjusted_logits(q, k)
    raw = sa_oracle.raw_logits(q, k)
    torch.testing.assert_close(logits.diagonal(-1, dim1=-2, dim2=-1), raw.diagonal(-1, dim1=-2, dim2=-1))


def test_reduces_to_causal_softmax_when_nothing_is_selected():
    """Negating head 0's k makes every L_0 <= 0 for q0 = -k0 patterns... here: head 0's q is the
    negative of a positive combination so q0.k0 < 0 for all pairs; and exempt >= T. Both reduce the
    operator to plain causal softmax attention (torch SDPA)."""
    q, k, v = _qkv(2, 3, 40, 16, seed=3)
    want = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    torch.testing.assert_close(sa_oracle.attention(q, k, v, exempt=40), want, atol=1e-12, rtol=1e-10)
    k0 = k.clone()
    k0[:, 0] = k0[:, 0].abs()
    q0 = q.clone()
    q0[:, 0] = -q0[:, 0].abs()
    want0 = F.scaled_dot_product_attention(q0, k0, v, is_causal=True)
    torch.testing.assert_close(sa_oracle.attention(q0, k0, v), want0, atol=1e-12, rtol=1e-10)


def test_attention_rows_sum_to_one():
    q, k, _ = _qkv(2, 2, 33, 8, seed=4, scale=2.0)
    logits, _ = sa_oracle.adjusted_logits(q, k)
    torch.testing.assert_close(logits.softmax(-1).sum(-1), torch.ones(2, 2, 33, dtype=torch.float64))


def test_analytic_backward_matches_autograd():
    q, k, v = _qkv(2, 3, 29, 8, seed=5, scale=1.5)
    dout = torch.randn(2, 3, 29, 8, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    (sa_oracle.attention(qq, kk, vv) * dout).sum().backward()
    dq, dk, dv = sa_oracle.backward(q, k, v, dout)
    torch.testing.assert_close(dq, qq.grad, atol=1e-12, rtol=1e-10)
    torch.testing.assert_close(dk, kk.grad, atol=1e-12, rtol=1e-10)
    torch.testing.assert_close(dv, vv.grad, atol=1e-12, rtol=1e-10)


def test_autograd_matches_finite_differences():
    q, k, v = _qkv(1, 2, 7, 4, seed=6, scale=1.5)
    assert torch.autograd.gradcheck(lambda a, b, c: sa_oracle.attention(a, b, c),
                                    tuple(t.clone().requires_grad_(True) for t in (q, k, v)))


def test_a_dropped_selection_term_is_caught():
    """Planted mistake: computing F from inclusive instead of exclusive prefixes must fail the loop pin."""
    q, k, v = _qkv(1, 2, 15, 8, seed=7, scale=2.0)
    sel = sa_oracle.selection(q, k)
    wrong = sa_oracle.raw_logits(q, k) - torch.cumsum(sel, dim=-2)[:, None]
    wrong = wrong.masked_fill(~torch.ones(15, 15, dtype=torch.bool).tril(), float("-inf"))
    out_loop, _ = sa_oracle.attention_loop(q, k, v)
    assert (wrong.softmax(-1) @ v - out_loop).abs().max() > 1e-3


def test_head_zero_gets_gradient_only_through_history():
    """reference tests/test_selective_kernels.py:88-100 (oracle side)"""
    q, k, v = _qkv(1, 3, 40, 8, seed=3, scale=2.0)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    sa_oracle.attention(qq, kk, vv)[:, 1:].sum().backward()
    assert qq.grad[:, 0].abs().max() > 1e-4 and vv.grad[:, 0].abs().max() == 0


@pytest.mark.parametrize("chunk", [1, 7, 16, 64])
def test_prefill_chunks_equal_single_shot(chunk):
    q, k, v = _qkv(2, 2, 50, 8, seed=chunk, scale=1.5)
    out, state = sa_oracle.prefill_chunks(q, k, v, chunk)
    torch.testing.assert_close(out, sa_oracle.attention(q, k, v), atol=1e-12, rtol=1e-10)
    torch.testing.assert_close(state, sa_oracle.selection_totals(q, k), atol=1e-12, rtol=1e-10)


def test_tail_equals_last_rows():
    q, k, v = _qkv(1, 2, 90, 8, seed=8, scale=1.5)
    rows, out, total = sa_oracle.tail(q, k, v, 20, chunk=16)
    torch.testing.assert_close(out, sa_oracle.attention(q, k, v)[:, :, rows], atol=1e-12, rtol=1e-10)
    torch.testing.assert_close(total, sa_oracle.selection_totals(q, k), atol=1e-12, rtol=1e-10)


def test_decode_steps_equal_single_shot():
    """reference tests/test_selective_model.py:42-53 (operator level)"""
    q, k, v = _qkv(2, 3, 30, 8, seed=9, scale=1.5)
    out, state = sa_oracle.decode_steps(q, k, v, prompt=12)
    torch.testing.assert_close(out, sa_oracle.attention(q, k, v)[:, :, 12:], atol=1e-12, rtol=1e-10)
    torch.testing.assert_close(state, sa_oracle.selection_totals(q, k), atol=1e-12, rtol=1e-10)


def test_decode_step_from_arbitrary_state():
    """One step from a random non-negative state, against the softmax written out per key with exp
    and sums, and the state update written per key (head 0's relu logit on keys [E, t-1))."""
    q, k, v = _qkv(2, 3, 17, 8, seed=15, scale=1.5)
    g = torch.Generator().manual_seed(16)
    state = torch.rand(2, 20, generator=g, dtype=torch.float64) * 3
    out, new_state = sa_oracle.decode_step(q[:, :, -1:], k, v, state, exempt=2)
    s = 1 / math.sqrt(8)
    for b in range(2):
        for h in range(3):
            z = [s * float(q[b, h, -1] @ k[b, h, j]) - float(state[b, j]) for j in range(17)]
            w = [math.exp(x - max(z)) for x in z]
            want = sum(wj * v[b, h, j] for j, wj in enumerate(w)) / sum(w)
            torch.testing.assert_close(out[b, h, 0], want, atol=1e-12, rtol=1e-10)
        for j in range(20):
            raw0 = s * float(q[b, 0, -1] @ k[b, 0, j]) if j < 17 else 0.0
            add = max(raw0, 0.0) if 2 <= j < 16 else 0.0
            assert abs(float(new_state[b, j]) - (float(state[b, j]) + add)) < 1e-12


def test_per_head_equals_each_head_alone():
    """reference tests/test_selective_perhead.py:25-29"""
    q, k, v = _qkv(2, 3, 21, 8, seed=10, scale=1.5)
    got = sa_oracle.per_head(q, k, v)
    for h in range(3):
        sl = slice(h, h + 1)
        torch.testing.assert_close(got[:, sl], sa_oracle.attention(q[:, sl], k[:, sl], v[:, sl]))


def test_oracle_rejects_exempt_zero():
    q, k, v = _qkv(1, 1, 8, 16)
    with pytest.raises(ValueError, match="exempt"):
        sa_oracle.attention(q, k, v, exempt=0)


# -- the package's exported listing (selective_logits / selective_attention_reference) ------------

@pytest.mark.parametrize("exempt", [1, 3])
def test_package_listing_matches_oracle(exempt):
    q, k, v = _qkv(2, 3, 37, 16, seed=11, scale=1.5, dtype=torch.float32)
    got = kernels.selective_attention_reference(q, k, v, exempt)
    want = sa_oracle.attention(q.double(), k.double(), v.double(), exempt)
    torch.testing.assert_close(got.double(), want, atol=1e-5, rtol=1e-5)
    logits, total = kernels.selective_logits(q, k, exempt)
    wl, wt = sa_oracle.adjusted_logits(q.double(), k.double(), exempt)
    torch.testing.assert_close(logits.double(), wl, atol=1e-4, rtol=1e-5)
    torch.testing.assert_close(total.double(), wt, atol=1e-4, rtol=1e-5)


def test_package_listing_rejects_exempt_zero():
    q, k, v = _qkv(1, 1, 8, 16, dtype=torch.float32)
    with pytest.raises(ValueError, match="exempt"):
        kernels.selective_attention_reference(q, k, v, exempt=0)
