"""The allocation-free decode entry point (sa_decode_noalloc: the step's scratch in the library's
fixed device array, no workspace argument) against sa_decode with a caller workspace, both called
through the C ABI on the same inputs: outputs and state updates identical, over two calls in a row
(the second smaller, so it runs over what the first left in the array), shared and per-head
selection, bf16 and fp32 caches."""

from __future__ import annotations

import pytest
import torch

from selective_attention import _lib

pytestmark = pytest.mark.gpu

CASES = [
    # (nseq, heads, groups, t, head_dim, dtype): the second call of each pair is smaller
    ((2, 16, 1, 70001, 64, torch.bfloat16), (1, 4, 1, 300, 64, torch.bfloat16)),
    ((1, 8, 8, 20000, 128, torch.float32), (1, 2, 2, 1000, 32, torch.float32)),
]


def _step(cuda, nseq, heads, groups, t, head_dim, dtype, seed, noalloc):
    """One decode step through the C ABI; returns (out, state after the step)."""
    lib = _lib.load()
    g = torch.Generator(device=cuda).manual_seed(seed)
    q = torch.randn(nseq * heads, head_dim, device=cuda, generator=g).to(dtype)
    k = torch.randn(nseq * heads, t, head_dim, device=cuda, generator=g).to(dtype)
    v = torch.randn(nseq * heads, t, head_dim, device=cuda, generator=g).to(dtype)
    state_ld = t + 5
    sel = torch.rand(nseq * groups, state_ld, device=cuda, generator=g)
    out = torch.full((nseq * heads, head_dim), float("nan"), device=cuda)
    code = _lib.DTYPE_BF16 if dtype == torch.bfloat16 else _lib.DTYPE_F32
    scale = head_dim ** -0.5
    stream = torch.cuda.current_stream(cuda).cuda_stream
    with torch.cuda.device(cuda):
        if noalloc:
            before = torch.cuda.memory_allocated(cuda)
            rc = lib.sa_decode_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), sel.data_ptr(),
                                       state_ld, nseq, heads, groups, t, 0, head_dim, scale, code, 1, stream)
            assert torch.cuda.memory_allocated(cuda) == before
        else:
            nbytes = int(lib.sa_decode_workspace_bytes(nseq, heads, t, head_dim))
            ws = torch.empty(nbytes, device=cuda, dtype=torch.uint8)
            rc = lib.sa_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), sel.data_ptr(), state_ld,
                               ws.data_ptr(), nbytes, nseq, heads, groups, t, 0, head_dim, scale, code, 1, stream)
    _lib.check(rc)
    torch.cuda.synchronize(cuda)
    return out, sel


@pytest.mark.parametrize("pair", CASES, ids=["bf16-shared", "f32-per-head"])
def test_noalloc_decode_equals_workspace_decode(cuda, pair):
    for i, shape in enumerate(pair):
        print(f"case noalloc decode call {i}: (nseq, heads, groups, t, D, dtype) = {shape}", flush=True)
        want_out, want_sel = _step(cuda, *shape, seed=100 + i, noalloc=False)
        got_out, got_sel = _step(cuda, *shape, seed=100 + i, noalloc=True)
        assert torch.isfinite(got_out).all()
        assert torch.equal(got_out, want_out)
        assert torch.equal(got_sel, want_sel)
