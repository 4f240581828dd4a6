"""Repeated calls on the same inputs give the same bits: every kernel on the path writes each output
element from one wavefront in a fixed order, and head 0's dQ / dK, which gather a share from every
head group, take those shares from one workspace slot per group, summed in group order (no atomics),
so any difference between two runs is a race -- an LDS buffer read before its direct load landed,
or overwritten while still read. The reference's backward is not
deterministic in this sense: it adds dQ per key block with relaxed fp32 atomics
(src/selective_attention/kernels.py:257, 283), where this build's query side owns each dQ row and
stores it once.

The shapes put every kernel instance of the bf16 head-dim-64 path to work: two heads per wavefront
in the forward and the multi-head backward kernels (B=1, H=4, T=2048), one head per wavefront with
many sequences (the per-head mode: the one-pass selection carry, the one-head forward and backward
instances), and a chunked prefill (the forward over a strided key / value view with a carried
state)."""

from __future__ import annotations

import pytest
import torch

from selective_attention import kernels

pytestmark = pytest.mark.gpu

REPEATS = 4


def _inputs(shape, seed, cuda):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(*shape, generator=g).bfloat16().to(cuda) for _ in range(4)]


def _fwd_bwd(q, k, v, do, exempt=1):
    qs, ks, vs = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
    out = kernels.selective_attention(qs, ks, vs, exempt=exempt)
    out.backward(do.float())
    return out.detach(), qs.grad, ks.grad, vs.grad


def _other_work(cuda):
    """A fwd+bwd of another shape between repeats: LDS and the allocator's blocks then hold what
    other kernels left, so a result that depends on state from earlier launches (a read of LDS its
    own loads had not filled) differs between repeats instead of repeating itself."""
    q, k, v, do = _inputs((2, 4, 1536, 64), seed=77, cuda=cuda)
    _fwd_bwd(q, k, v, do)


@pytest.mark.parametrize("shape", [(1, 4, 2048, 64), (32, 1, 1024, 64)], ids=["heads", "per_head"])
def test_repeated_fwd_bwd_is_bit_identical(cuda, shape):
    print(f"case determinism fwd+bwd {shape}", flush=True)
    q, k, v, do = _inputs(shape, seed=sum(shape), cuda=cuda)
    first = _fwd_bwd(q, k, v, do)
    for i in range(REPEATS - 1):
        if i % 2 == 0:
            _other_work(cuda)
        again = _fwd_bwd(q, k, v, do)
        # every output bit for bit, head 0's dQ, dK (the multi-head shape's share slots and their
        # fixed-order sum) included
        for a, b in zip(first, again):
            assert torch.equal(a, b)


@pytest.mark.parametrize("dtype,head_dim,heads", [(torch.bfloat16, 32, 6), (torch.float32, 64, 3), (torch.bfloat16, 128, 3)],
                         ids=["bf16_d32_groups_of_2", "fp32_d64", "bf16_d128"])
def test_repeated_generic_backward_is_bit_identical(cuda, dtype, head_dim, heads):
    """The other backward instances (two heads per wavefront at bf16 head dim 32, fp32 storage, head
    dim 128) sum head 0's shares from their group slots the same way: bit for bit."""
    print(f"case determinism generic backward {dtype} D={head_dim} H={heads}", flush=True)
    g = torch.Generator().manual_seed(head_dim + heads)
    q, k, v, do = (torch.randn(2, heads, 333, head_dim, generator=g).to(dtype).to(cuda) for _ in range(4))
    runs = []
    for i in range(3):
        if i == 1:
            _other_work(cuda)
        runs.append(_fwd_bwd(q, k, v, do))
    for again in runs[1:]:
        for a, b in zip(runs[0], again):
            assert torch.equal(a, b)


@pytest.mark.parametrize("n", [128, 8], ids=["one_pass", "two_kernel"])
def test_repeated_forward_with_carry_is_bit_identical(cuda, n):
    """The per-head forward and its aux outputs over one-head sequences of a ragged length: 128 of
    them take the one-pass selection carry, 8 the column sums and scan (a grid too small for the one
    pass)."""
    print(f"case determinism forward carry n={n}", flush=True)
    q, k, v, _ = _inputs((n, 1, 2047, 64), seed=5, cuda=cuda)
    runs = []
    for i in range(2 * REPEATS):
        if i % 2:
            _other_work(cuda)
        runs.append(kernels.selective_attention_forward(q, k, v, exempt=16, return_aux=True))
    for out, aux in runs[1:]:
        assert torch.equal(runs[0][0], out)
        assert torch.equal(runs[0][1]["carry"], aux["carry"])
        assert torch.equal(runs[0][1]["selected_total"], aux["selected_total"])


def test_repeated_chunked_prefill_is_bit_identical(cuda):
    print("case determinism chunked prefill", flush=True)
    q, k, v, _ = _inputs((64, 1, 1024, 64), seed=9, cuda=cuda)
    results = []
    for i in range(REPEATS):
        if i % 2:
            _other_work(cuda)
        state = torch.zeros(64, 1024, device=cuda)
        outs = [kernels.selective_attention_prefill(q[:, :, c0:c0 + 256], k[:, :, :c0 + 256], v[:, :, :c0 + 256],
                                                    state, c0) for c0 in range(0, 1024, 256)]
        results.append((torch.cat(outs, dim=2), state))
    for out, state in results[1:]:
        assert torch.equal(results[0][0], out)
        assert torch.equal(results[0][1], state)


def test_batched_equals_each_sequence_alone(cuda):
    """A sequence's outputs and gradients do not depend on what else shares its launch: 8 sequences of
    12 heads in one call equal each sequence run alone, bit for bit. The batched call is sized so that
    its query-side backward holds 2.7-3 workgroups per CU slot, where that kernel deals its workgroups
    to the XCDs in the order of work_order_block(slots) (shortest third after the first round); the
    single-sequence calls fill less than one round and take the longest-first order, and their
    forward runs one head per wavefront where the batched one runs two. A dispatch order that lost or
    repeated a workgroup, or a result that depended on the order, would show here."""
    b, h, t, d = 8, 12, 2048, 64
    cus = torch.cuda.get_device_properties(cuda).multi_processor_count
    rounds = (t // 256) * b * h / ((cus // 8) * 8)
    print(f"case batched vs alone B={b} H={h} T={t}: query-side rounds {rounds:.2f}", flush=True)
    assert 2.7 <= rounds <= 3.0, rounds   # (the regime this test is for, on an MI355X's 256 CUs)
    q, k, v, do = _inputs((b, h, t, d), seed=12, cuda=cuda)
    whole = _fwd_bwd(q, k, v, do)
    for i in range(b):
        sl = slice(i, i + 1)
        alone = _fwd_bwd(q[sl].contiguous(), k[sl].contiguous(), v[sl].contiguous(), do[sl].contiguous())
        for name, x, y in zip(("out", "dq", "dk", "dv"), whole, alone):
            assert torch.equal(x[sl], y), (i, name)
