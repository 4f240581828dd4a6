"""The packed-projection form (selective_attention_qkv, sa_forward_strided / sa_backward_strided):
q, k, v read in place from a (B, T, 3 * H * D) projection, the output written as (B, T, H * D) in
the projection's dtype, the gradient as one (B, T, 3 * H * D) tensor. It runs the same kernels as
selective_attention on the split heads, so outputs and gradients must equal that path's exactly
(output cast to the projection's dtype and merged, gradients assembled from the slices), and the
fp64 oracle to the usual bound."""

from __future__ import annotations

import pytest
import torch

from oracle import sa_oracle
from selective_attention import kernels

pytestmark = pytest.mark.gpu


def _split(qkv, heads):
    b, t, c3 = qkv.shape
    d = c3 // (3 * heads)
    x = qkv.view(b, t, 3, heads, d)
    return tuple(x[:, :, i].transpose(1, 2) for i in range(3))


def _reference_path(qkv, heads, dy, dot_precision, exempt):
    """selective_attention on the split heads, merged as the attention slot does."""
    x = qkv.detach().clone().requires_grad_(True)
    q, k, v = _split(x, heads)
    o = kernels.selective_attention(q, k, v, dot_precision=dot_precision, exempt=exempt).to(x.dtype)
    y = o.transpose(1, 2).reshape(x.shape[0], x.shape[1], -1)
    y.backward(dy)
    return y.detach(), x.grad


@pytest.mark.parametrize("dtype,dot_precision", [(torch.bfloat16, None), (torch.float32, "ieee")])
@pytest.mark.parametrize("head_dim,heads,t,exempt", [(64, 4, 300, 1), (32, 3, 129, 3), (128, 2, 200, 1)])
def test_packed_equals_split_heads(cuda, dtype, dot_precision, head_dim, heads, t, exempt):
    print(f"case packed {dtype} D={head_dim} H={heads} T={t} E={exempt}", flush=True)
    g = torch.Generator().manual_seed(21)
    b = 2
    qkv = torch.randn(b, t, 3 * heads * head_dim, generator=g).to(dtype).to(cuda)
    dy = torch.randn(b, t, heads * head_dim, generator=g).to(dtype).to(cuda)
    want_y, want_g = _reference_path(qkv, heads, dy, dot_precision, exempt)
    x = qkv.detach().clone().requires_grad_(True)
    y = kernels.selective_attention_qkv(x, heads, dot_precision=dot_precision, exempt=exempt)
    y.backward(dy)
    assert y.dtype == dtype and y.shape == (b, t, heads * head_dim)
    torch.testing.assert_close(y, want_y, rtol=0, atol=0)
    # exact, head 0's dQ and dK included (the other head groups' shares of them are summed in a
    # fixed order from one slot per group)
    torch.testing.assert_close(x.grad, want_g, rtol=0, atol=0)


def test_packed_matches_oracle(cuda):
    """Absolute parity: output and gradients against the fp64 listing (bf16 operands: 2e-2, plus
    1e-2 relative for the bf16 rounding of the returned values themselves)."""
    g = torch.Generator().manual_seed(22)
    b, t, heads, d = 1, 257, 4, 64
    qkv = torch.randn(b, t, 3 * heads * d, generator=g).bfloat16()
    dy = torch.randn(b, t, heads * d, generator=g).bfloat16()
    x = qkv.to(cuda).requires_grad_(True)
    y = kernels.selective_attention_qkv(x, heads)
    y.backward(dy.to(cuda))
    q, k, v = (z.double().contiguous() for z in _split(qkv, heads))
    want = sa_oracle.attention(q, k, v)
    torch.testing.assert_close(y.float().cpu().double(), want.transpose(1, 2).reshape(b, t, -1), atol=2e-2,
                               rtol=1e-2)
    do4 = dy.double().view(b, t, heads, d).transpose(1, 2)
    dq, dk, dv = sa_oracle.backward(q, k, v, do4)
    got = x.grad.float().cpu().double().view(b, t, 3, heads, d)
    for i, w in enumerate((dq, dk, dv)):
        torch.testing.assert_close(got[:, :, i].transpose(1, 2), w, atol=2e-2, rtol=1e-2)


def test_packed_rejects_what_it_cannot_read(cuda):
    qkv = torch.randn(1, 16, 3 * 4 * 64, device=cuda, dtype=torch.float16)
    assert not kernels.packed_supported(qkv, 4)              # fp16 is stored as fp32: not in place
    with pytest.raises(ValueError, match="dtype"):
        kernels.selective_attention_qkv(qkv, 4)
    assert not kernels.packed_supported(torch.randn(1, 16, 3 * 4 * 16, device=cuda, dtype=torch.bfloat16), 4)
    assert kernels.packed_supported(qkv.bfloat16(), 4)
