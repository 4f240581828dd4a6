"""GPU parity of the selection pass (reference src/selective_attention/kernels.py:112-138,
`_selective_carry`: each key's running selection, stored on entry to every 32-query block, and the
totals over all queries).

The library takes two paths to it: column sums over query blocks then a scan (calls with few
sequences), or one pass per key block that walks every query block (calls with sequences enough to
fill the GPU, the per-head mode's shape). Both add each block's sum in the same order, so on the
same sequences they agree bit for bit; the carry checkpoints and totals are also checked against
the oracle's history (fp64 on the same bf16-rounded inputs).
"""

from __future__ import annotations

import pytest
import torch

from oracle import sa_oracle
from selective_attention import kernels

pytestmark = pytest.mark.gpu

# the one-pass kernel runs when ceil(ceil(T/32)/4) x sequences >= 256 workgroups
ONE_PASS_WORKGROUPS = 256


def _workgroups(n, t):
    return -(-(-(-t // 32)) // 4) * n


def _seqs(n, t, seed):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(n, 1, t, 64, generator=g).bfloat16() for _ in range(3))


def _forward(q, k, v, cuda, exempt):
    out, aux = kernels.selective_attention_forward(q.to(cuda), k.to(cuda), v.to(cuda), exempt=exempt,
                                                   return_aux=True)
    return out, aux["carry"], aux["selected_total"]


@pytest.mark.parametrize("t,exempt", [(2048, 1), (2047, 16), (1985, 1)])
def test_one_pass_carry_equals_two_kernel_path(cuda, t, exempt):
    n = 128
    assert _workgroups(n, t) >= ONE_PASS_WORKGROUPS and _workgroups(8, t) < ONE_PASS_WORKGROUPS
    print(f"case one-pass selection t={t} exempt={exempt}", flush=True)
    q, k, v = _seqs(n, t, seed=t + exempt)
    out1, carry1, total1 = _forward(q, k, v, cuda, exempt)          # one pass over 128 sequences
    parts = [_forward(q[i:i + 8], k[i:i + 8], v[i:i + 8], cuda, exempt) for i in range(0, n, 8)]
    assert torch.equal(carry1, torch.cat([p[1] for p in parts]))
    assert torch.equal(total1, torch.cat([p[2] for p in parts]))
    assert torch.equal(out1, torch.cat([p[0] for p in parts]))

    # against the oracle on a few sequences: carry[rb] = the history at query rb*32
    for s in (0, n - 1):
        sel = sa_oracle.selection(q[s:s + 1, :1].double(), k[s:s + 1, :1].double(), exempt)   # (1, T, T)
        hist = sa_oracle.history(sel)
        want_carry = hist[:, ::32, :]
        torch.testing.assert_close(carry1[s:s + 1].cpu().double(), want_carry, rtol=1e-5, atol=1e-3)
        torch.testing.assert_close(total1[s:s + 1].cpu().double(), sel.sum(dim=-2), rtol=1e-5, atol=1e-3)


def test_one_pass_carry_continues_a_chunked_prefill(cuda):
    """Chunks whose key count puts them on the one-pass kernel carry state_in (keys before the chunk)
    and leave the same state and outputs as the two-kernel path."""
    n, t, chunk = 512, 1024, 256
    q, k, v = (x.to(cuda) for x in _seqs(n, t, seed=7))
    states = {}
    outs = {}
    for split in (n, 16):   # all 512 sequences per call, or 16 at a time (the two-kernel path)
        state = torch.zeros(n, t, device=cuda)
        got = []
        for c0 in range(0, t, chunk):
            print(f"case one-pass prefill split={split} c0={c0}", flush=True)
            part = [kernels.selective_attention_prefill(q[i:i + split, :, c0:c0 + chunk], k[i:i + split, :, :c0 + chunk],
                                                        v[i:i + split, :, :c0 + chunk], state[i:i + split], c0)
                    for i in range(0, n, split)]
            got.append(torch.cat(part))
        states[split], outs[split] = state, torch.cat(got, dim=2)
    assert _workgroups(n, t) >= ONE_PASS_WORKGROUPS > _workgroups(16, t)
    assert torch.equal(states[n], states[16])
    assert torch.equal(outs[n], outs[16])
    want = sa_oracle.selection_totals(q[:2].cpu().double(), k[:2].cpu().double())
    torch.testing.assert_close(states[n][:2].cpu().double(), want, rtol=1e-5, atol=1e-3)
