"""The cached decode step on the GPU (reference mixers.py:115-130, `SelectiveAttention.step_cache`):
the HIP kernel's outputs and selection-state updates against the oracle's one-query-at-a-time
decode (`oracle.sa_oracle.decode_steps`, itself pinned against the single-shot forward), for the
shared variant (head 0 selects) and the per-head variant (every head selects for itself)."""

from __future__ import annotations

import pytest
import torch

from oracle import sa_oracle
from selective_attention import kernels

pytestmark = pytest.mark.gpu


def _inputs(b, h, t, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(b, h, t, d, generator=g).to(dtype) for _ in range(3))


def _cache(x, cap, cuda):
    c = torch.zeros(x.shape[0], x.shape[1], cap, x.shape[3], dtype=x.dtype, device=cuda)
    c[:, :, : x.shape[2]] = x.to(cuda)
    return c


def _tol(dtype):
    # both sides compute in fp32 / fp64 on the same (bf16-representable) operand values
    return dict(atol=2e-5, rtol=2e-5) if dtype == torch.float32 else dict(atol=3e-5, rtol=3e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [32, 64, 128])
@pytest.mark.parametrize("exempt", [1, 3])
def test_shared_decode_steps_match_oracle(cuda, dtype, head_dim, exempt):
    """Steps 250..299 (crossing the kernel's 256-key chunk boundary) after a 250-token prompt."""
    print(f"case shared decode {dtype} D={head_dim} exempt={exempt}", flush=True)
    b, h, t, prompt = 2, 4, 300, 250
    q, k, v = _inputs(b, h, t, head_dim, dtype, 11)
    want, want_state = sa_oracle.decode_steps(q.double(), k.double(), v.double(), prompt, exempt)
    _, state0 = sa_oracle.prefill_chunks(q[:, :, :prompt].double(), k[:, :, :prompt].double(),
                                         v[:, :, :prompt].double(), prompt, exempt)
    cap = t + 7
    kc, vc = _cache(k, cap, cuda), _cache(v, cap, cuda)
    sel = torch.zeros(b, 1, cap, device=cuda)
    sel[:, 0, :prompt] = state0.float().to(cuda)
    outs = [kernels.selective_attention_decode(q[:, :, i].to(cuda), kc[:, :, : i + 1], vc[:, :, : i + 1], sel,
                                               exempt=exempt) for i in range(prompt, t)]
    got = torch.stack(outs, dim=2).cpu().double()
    torch.testing.assert_close(got, want, **_tol(dtype))
    torch.testing.assert_close(sel[:, 0, :t].cpu().double(), want_state, **_tol(dtype))
    assert not sel[:, 0, t:].any()   # past the current length the state is untouched


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_per_head_decode_steps_match_oracle(cuda, dtype):
    """Every head its own selector (groups = heads): each head as its own one-head sequence."""
    b, h, t, prompt, d = 2, 3, 140, 120, 64
    q, k, v = _inputs(b, h, t, d, dtype, 12)
    r = lambda x: x.reshape(b * h, 1, t, d).double()
    want, want_state = sa_oracle.decode_steps(r(q), r(k), r(v), prompt)
    _, state0 = sa_oracle.prefill_chunks(r(q)[:, :, :prompt], r(k)[:, :, :prompt], r(v)[:, :, :prompt], prompt)
    cap = t
    kc, vc = _cache(k, cap, cuda), _cache(v, cap, cuda)
    sel = torch.zeros(b, h, cap, device=cuda)
    sel[:, :, :prompt] = state0.float().reshape(b, h, prompt).to(cuda)
    outs = [kernels.selective_attention_decode(q[:, :, i].to(cuda), kc[:, :, : i + 1], vc[:, :, : i + 1], sel)
            for i in range(prompt, t)]
    got = torch.stack(outs, dim=2).cpu().double()
    torch.testing.assert_close(got, want.reshape(b, h, t - prompt, d), **_tol(dtype))
    torch.testing.assert_close(sel.cpu().double(), want_state.reshape(b, h, t), **_tol(dtype))


def test_long_cache_single_step(cuda):
    """One step at t = 2100 (nine 256-key chunks, a partial last one) with a non-trivial state."""
    b, h, t, d = 1, 2, 2100, 64
    q, k, v = _inputs(b, h, t, d, torch.bfloat16, 13)
    want, want_state = sa_oracle.decode_steps(q.double(), k.double(), v.double(), t - 1)
    _, state0 = sa_oracle.prefill_chunks(q[:, :, : t - 1].double(), k[:, :, : t - 1].double(),
                                         v[:, :, : t - 1].double(), t - 1)
    kc, vc = _cache(k, t, cuda), _cache(v, t, cuda)
    sel = torch.zeros(b, 1, t, device=cuda)
    sel[:, 0, : t - 1] = state0.float().to(cuda)
    got = kernels.selective_attention_decode(q[:, :, t - 1].to(cuda), kc, vc, sel)
    torch.testing.assert_close(got[:, :, None].cpu().double(), want, atol=3e-5, rtol=3e-5)
    torch.testing.assert_close(sel[:, 0].cpu().double(), want_state, atol=3e-5, rtol=3e-5)


@pytest.mark.parametrize("dtype,head_dim,heads,t", [(torch.bfloat16, 64, 2, 70001), (torch.float32, 128, 1, 33000),
                                                     (torch.bfloat16, 32, 16, 20000)])
def test_many_partials_single_step(cuda, dtype, head_dim, heads, t):
    """One step over a long cache from a random state (oracle.decode_step): hundreds of workgroup
    partials per head, more than the merge kernel takes in one pass."""
    print(f"case long decode {dtype} D={head_dim} H={heads} t={t}", flush=True)
    g = torch.Generator().manual_seed(17)
    q, k, v = (torch.randn(1, heads, t, head_dim, generator=g).to(dtype) for _ in range(3))
    state = torch.rand(1, t + 3, generator=g) * 4
    want, want_state = sa_oracle.decode_step(q[:, :, -1:].double(), k.double(), v.double(), state.double())
    sel = state[:, None].to(cuda)
    got = kernels.selective_attention_decode(q[:, :, -1].to(cuda), k.to(cuda), v.to(cuda), sel)
    torch.testing.assert_close(got[:, :, None].cpu().double(), want, **_tol(dtype))
    torch.testing.assert_close(sel[:, 0].cpu().double(), want_state, atol=2e-5, rtol=2e-5)


def test_decode_rejects_bad_state(cuda):
    q, k, v = (x.to(cuda) for x in _inputs(1, 4, 10, 64, torch.bfloat16, 14))
    with pytest.raises(ValueError, match="selected"):
        kernels.selective_attention_decode(q[:, :, -1], k, v, torch.zeros(1, 3, 10, device=cuda))   # 3 does not divide 4
    with pytest.raises(ValueError, match="selected"):
        kernels.selective_attention_decode(q[:, :, -1], k, v, torch.zeros(1, 1, 9, device=cuda))    # shorter than t
