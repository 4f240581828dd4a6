"""Selective Attention on MI355X: the reference's operator API over hand-written gfx950 HIP kernels.

Selective Attention (Leviathan, Kalman, Matias, "Selective Attention Improves Transformer",
ICLR 2025) is causal softmax attention with one extra term on the logits:

    L_h[i, j] = q_h[i] . k_h[j] / sqrt(D)                    # every head h, key j <= query i
    S[i, j]   = relu(L_0[i, j])     for E <= j < i, else 0   # head 0 only; E = `exempt` (1: <BOS>)
    F[i, j]   = sum over r < i of S[r, j]
    A_h       = causal_softmax(L_h - F);   out_h = A_h @ v_h

This module keeps the names, keyword arguments and error messages of the reference's
`selective_attention.kernels` (reference src/selective_attention/kernels.py:61-83, 427-703) so
callers switch by import path. The work runs in libsa_hip.so (include/sa.h):

    selection   column sums of head 0's S per 32-query block, then an exclusive running sum:
                CARRY (B, ceil(T/32), T) fp32, the reference's checkpoint layout, plus the totals
    forward     query-parallel flash-style online softmax of L_h - F on bf16 (or fp32) MFMA
    backward    key-parallel reverse sweep with the selection suffix sum in registers

`dot_precision` picks the MFMA operand type: "bf16" (default for bf16 inputs) runs bf16
operands with fp32 accumulation; "tf32" (default otherwise) and "ieee" both run fp32 operands on
fp32 MFMA, since gfx950 has no TF32 datapath (so "tf32" is exact fp32 here). fp16 inputs are
converted to the operand type; outputs are fp32 as in the reference, gradients come back in the
input dtypes.

Tile and launch kwargs of the reference (block_m, block_n, num_warps, num_stages, bwd_block_n,
bwd_num_warps, bwd_num_stages) are accepted and validated as the reference does, but do not
change the launch: the HIP kernels use 32 x 32 MFMA tiles and 256-thread workgroups. `group`
(forward) and `bwd_group` (backward) set the heads per wavefront, within what the kernels
instantiate (results do not depend on them beyond fp32 summation order).

There is no silent fallback: on CUDA (ROCm) tensors the HIP library must load, or these
functions raise RuntimeError. `selective_logits` / `selective_attention_reference` are the plain
torch listing, exported as in the reference.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch.autograd.function import once_differentiable

from . import _lib

HAS_HIP = _lib.available()
# The reference's callers gate the fused path on `kernels.HAS_TRITON`; the same flag here means
# "the fused (HIP) kernels can run".
HAS_TRITON = HAS_HIP

# Query rows per CARRY checkpoint (reference kernels.py:87).
CARRY_M = 32
HEAD_DIMS = (16, 32, 64, 128)
DTYPES = (torch.float16, torch.bfloat16, torch.float32)


# -- the listing ----------------------------------------------------------------------------------

def selective_logits(q: torch.Tensor, k: torch.Tensor, exempt: int = 1) -> tuple[torch.Tensor, torch.Tensor]:
    """Adjusted logits L - F, (B, H, T, T) fp32 with -inf above the diagonal, and the selection each
    key has received from all T queries, (B, T) (reference kernels.py:61-76)."""

    exempt = _check_exempt(exempt)
    seq, head_dim = q.shape[-2], q.shape[-1]
    logits = (q.float() @ k.float().transpose(-2, -1)) / math.sqrt(head_dim)
    pos = torch.arange(seq, device=q.device)
    logits = logits.masked_fill(pos[None, :] > pos[:, None], float("-inf"))
    # head 0 selects key j from query r when exempt <= j < r and its logit is positive
    selectable = (pos[None, :] < pos[:, None]) & (pos[None, :] >= exempt)
    sel = torch.where(selectable, torch.relu(logits[:, 0]), torch.zeros((), device=q.device))
    total = sel.sum(dim=-2)
    history = torch.zeros_like(sel)
    history[..., 1:, :] = torch.cumsum(sel, dim=-2)[..., :-1, :]   # strictly earlier queries
    return logits - history[:, None], total


def selective_attention_reference(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, exempt: int = 1) -> torch.Tensor:
    """Selective Attention written plainly (fp32). q / k / v: (B, H, T, D). Returns (B, H, T, D)
    (reference kernels.py:79-83)."""

    return selective_logits(q, k, exempt)[0].softmax(dim=-1) @ v.float()


# -- input checks and launch policy ----------------------------------------------------------------

def _resolve_precision(dot_precision: str | None, dtype: torch.dtype) -> int:
    """The operand storage of the kernels: _lib.DTYPE_BF16 or _lib.DTYPE_F32
    (reference kernels.py:427-437)."""

    if dot_precision is None:
        dot_precision = "bf16" if dtype == torch.bfloat16 else "tf32"
    if dot_precision == "bf16":
        return _lib.DTYPE_BF16
    if dot_precision in ("ieee", "tf32"):
        return _lib.DTYPE_F32
    raise ValueError(f"dot_precision must be None, 'bf16', 'tf32' or 'ieee', not {dot_precision!r}")


def check_inputs(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """Raise ValueError / RuntimeError unless the kernels can run on these inputs
    (reference kernels.py:444-458)."""

    if not HAS_HIP:
        _lib.load()   # raises RuntimeError with the reason
    if q.dim() != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"q, k, v must all be (B, H, T, D); got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.is_cuda and k.device == q.device and v.device == q.device):
        raise ValueError("q, k, v must be CUDA (ROCm) tensors on one device")
    if any(t.dtype not in DTYPES for t in (q, k, v)):
        raise ValueError(f"dtype must be float16, bfloat16 or float32; got {q.dtype}, {k.dtype}, {v.dtype}")
    if q.shape[-1] not in HEAD_DIMS:
        raise ValueError(f"head_dim must be one of {HEAD_DIMS}; got {q.shape[-1]}")
    if q.shape[-2] < 1:
        raise ValueError("the sequence is empty")


def supported(q: torch.Tensor, k: torch.Tensor | None = None, v: torch.Tensor | None = None) -> bool:
    """True when check_inputs would pass (k and v default to q's shape and device)."""

    try:
        check_inputs(q, q if k is None else k, q if v is None else v)
    except (ValueError, RuntimeError):
        return False
    return True


def _check_exempt(exempt: int) -> int:
    if int(exempt) != exempt or exempt < 1:
        raise ValueError(f"exempt must be an integer >= 1 (position 0, <BOS>, is always exempt); got {exempt}")
    return int(exempt)


def _check_blocks(block_m: int | None, block_n: int) -> None:
    if (block_m is not None and block_m % CARRY_M) or block_n % CARRY_M:
        raise ValueError(f"block_m and block_n must be multiples of {CARRY_M}")


def _check_bwd_group(group) -> int:
    if group is None:
        return 0
    if group not in (1, 2):
        raise ValueError(f"bwd_group must be None, 1 or 2; got {group}")
    return int(group)


def _damp_mode(damp: str, train_len: int) -> int:
    mode = {"none": 0, "linear": 1, "sqrt": 2}.get(damp)
    if mode is None:
        raise ValueError(f"damp must be 'none', 'linear' or 'sqrt'; got {damp!r}")
    if mode and train_len < 1:
        raise ValueError("damp needs train_len (the trained context length)")
    return mode


def _kernel_dim(head_dim: int) -> int:
    """The C ABI runs head_dim 32, 64, 128; 16 is zero-padded to 32 (zero columns change neither
    q.k nor the kept output columns; the scale passed stays 1/sqrt(16))."""
    return 32 if head_dim < 32 else head_dim


def _storage(t: torch.Tensor, n: int, dtype: int, kdim: int) -> torch.Tensor:
    """(B, H, T, D) -> contiguous (B*H, T, kdim) in the operand storage dtype."""

    want = torch.bfloat16 if dtype == _lib.DTYPE_BF16 else torch.float32
    x = t.reshape(n, t.shape[-2], t.shape[-1])
    if x.dtype != want:
        x = x.to(want)
    if kdim != t.shape[-1]:
        x = F.pad(x, (0, kdim - t.shape[-1]))
    return x.contiguous()


def _kv_storage(t: torch.Tensor, n: int, dtype: int, kdim: int, allow_view: bool) -> tuple[torch.Tensor, int]:
    """(B, H, T, D) keys or values for sa_forward, and the element stride between heads. A view whose
    heads sit a fixed stride apart with contiguous (T, D) rows inside each head (a slice of a
    preallocated cache) is passed as is; anything else becomes contiguous first."""

    want = torch.bfloat16 if dtype == _lib.DTYPE_BF16 else torch.float32
    batch, heads, seq, head_dim = t.shape
    if allow_view and t.dtype == want and head_dim == kdim and t.stride(3) == 1 and t.stride(2) == head_dim:
        # flattened row r = b * heads + h must start at r * hs
        if heads > 1:
            hs = t.stride(1)
            rows_ok = batch == 1 or t.stride(0) == heads * hs
        else:
            hs = t.stride(0) if batch > 1 else seq * head_dim
            rows_ok = True
        if rows_ok and hs >= seq * head_dim and hs % 8 == 0 and t.data_ptr() % 16 == 0:
            return t, hs
    x = _storage(t, n, dtype, kdim)
    return x, seq * kdim


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _forward_launch(q, k, v, dtype, exempt, group, damp_mode, train_len, state_in=None, q_offset=0, state=None,
                    allow_view=True):
    """Run sa_forward on (B, H, Tq, D) q and (B, H, Tk, D) k, v; returns the padded fp32 output
    (B*H, Tq, kdim), rmax, rden, carry, the storage tensors and the state."""

    lib = _lib.load()
    batch, heads, tq, head_dim = q.shape
    tk = k.shape[-2]
    n = batch * heads
    kdim = _kernel_dim(head_dim)
    dev = q.device
    qs = _storage(q, n, dtype, kdim)
    ks, kstride = _kv_storage(k, n, dtype, kdim, allow_view)
    vs, vstride = _kv_storage(v, n, dtype, kdim, allow_view)
    if kstride != vstride:   # one stride serves both: fall back to contiguous copies
        ks, vs = _storage(k, n, dtype, kdim), _storage(v, n, dtype, kdim)
        kstride = tk * kdim
    nb = (tq + CARRY_M - 1) // CARRY_M
    out = torch.empty(n, tq, kdim, device=dev, dtype=torch.float32)
    rmax = torch.empty(n, tq, device=dev, dtype=torch.float32)
    rden = torch.empty(n, tq, device=dev, dtype=torch.float32)
    carry = torch.empty(batch, nb, tk, device=dev, dtype=torch.float32)
    if state is None:
        state = torch.empty(batch, tk, device=dev, dtype=torch.float32)
    ws_bytes = lib.sa_forward_workspace_bytes(batch, heads, tk, kdim, dtype)
    ws = torch.empty(max(int(ws_bytes), 1), device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        _lib.check(lib.sa_forward(
            qs.data_ptr(), ks.data_ptr(), vs.data_ptr(), out.data_ptr(), rmax.data_ptr(), rden.data_ptr(),
            carry.data_ptr(), None if state_in is None else state_in.data_ptr(), state.data_ptr(),
            state.stride(0), ws.data_ptr(), ws.numel(), batch, heads, tq, tk, q_offset, kstride, kdim,
            1.0 / math.sqrt(head_dim), dtype, exempt, group, damp_mode, train_len, _stream(dev)))
    return out, rmax, rden, carry, state, (qs, ks, vs)


def selective_attention_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dot_precision: str | None = None,
    block_m: int | None = None,
    block_n: int = 32,
    return_aux: bool = False,
    num_warps: int = 4,
    num_stages: int | None = None,
    group: int | None = None,
    exempt: int = 1,
    *,
    damp: str = "none",
    train_len: int = 0,
):
    """Fused forward, no autograd; returns fp32 outputs (B, H, T, D) (reference kernels.py:526-605).

    With return_aux=True also returns dict(rmax, rden, carry, selected_total): the row statistics
    (log2 domain), CARRY (B, ceil(T/32), T) and the selection every key received from all T queries
    (the cached-decode accumulator). damp ("none" | "linear" | "sqrt") with train_len scales the
    history term of query i by min(1, train_len / (i + 1)) (or its square root), evaluation only.
    """

    check_inputs(q, k, v)
    exempt = _check_exempt(exempt)
    dtype = _resolve_precision(dot_precision, q.dtype)
    _check_blocks(block_m, block_n)
    damp_mode = _damp_mode(damp, train_len)
    batch, heads, seq, head_dim = q.shape
    out, rmax, rden, carry, total, _ = _forward_launch(
        q, k, v, dtype, exempt, int(group or 0), damp_mode, int(train_len))
    result = out[..., :head_dim].reshape(batch, heads, seq, head_dim)
    if head_dim != out.shape[-1]:
        result = result.contiguous()
    if return_aux:
        return result, dict(rmax=rmax, rden=rden, carry=carry, selected_total=total)
    return result


def selective_attention_prefill(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    state: torch.Tensor,
    q_offset: int,
    dot_precision: str | None = None,
    exempt: int = 1,
    group: int | None = None,
) -> torch.Tensor:
    """One chunk of a chunked prefill (no reference counterpart: the reference runs long inputs as one
    forward with a T^2/8-byte CARRY, kernels.py:38-40).

    q: (B, H, Tc, D), the queries at absolute positions [q_offset, q_offset + Tc). k, v:
    (B, H, q_offset + Tc, D), every key and value so far. state: (B, L) fp32, L >= q_offset + Tc,
    holding for every key j < q_offset the selection received from all queries before q_offset;
    it is updated in place to cover the queries of this chunk too (entries >= q_offset are
    overwritten). Returns fp32 (B, H, Tc, D), equal to rows [q_offset, q_offset + Tc) of the
    single-shot forward.
    """

    if q.dim() != 4 or k.shape != v.shape or q.shape[:2] != k.shape[:2] or q.shape[-1] != k.shape[-1]:
        raise ValueError(f"q (B, H, Tc, D) and k, v (B, H, Tk, D) must all be 4-D with matching B, H, D; "
                         f"got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    check_inputs(q, q, q)
    check_inputs(k, k, v)
    exempt = _check_exempt(exempt)
    dtype = _resolve_precision(dot_precision, q.dtype)
    batch, heads, tc, head_dim = q.shape
    tk = k.shape[-2]
    if q_offset < 0 or q_offset + tc != tk:
        raise ValueError(f"k and v must hold q_offset + Tc = {q_offset + tc} positions; got {tk}")
    if (state.dim() != 2 or state.shape[0] != batch or state.shape[1] < tk or state.dtype != torch.float32
            or state.device != q.device or state.stride(1) != 1):
        raise ValueError(f"state must be a (B, >= {tk}) fp32 tensor with unit column stride on q's device")
    out, *_ = _forward_launch(q, k, v, dtype, exempt, int(group or 0), 0, 0,
                              state_in=state if q_offset > 0 else None, q_offset=int(q_offset), state=state)
    return out[..., :head_dim].reshape(batch, heads, tc, head_dim)


def selective_attention_decode(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    selected: torch.Tensor,
    exempt: int = 1,
) -> torch.Tensor:
    """One cached decode step through the HIP kernel (the reference runs this step as PyTorch ops,
    mixers.py:115-130): the newest query of every head, at position t-1, attends over the t cached
    keys (its own included) with the carried selection subtracted from its logits; then the
    selector head of every group adds this query's own selection to ``selected`` (in place).

    q: (B, H, 1, D) or (B, H, D). k, v: (B, H, t, D) (a slice of a preallocated cache is used in
    place). selected: (B, G, L) fp32, L >= t, G dividing H: group g's heads are g*H/G ... and its
    selector is the first of them (G = 1: head 0 selects for every head; G = H: every head for
    itself). Logits, softmax and sums are fp32 on the upcast operands, as the reference's step.
    Returns fp32 (B, H, D).
    """

    if q.dim() == 4:
        if q.shape[2] != 1:
            raise ValueError(f"decode takes one query per head; got q of shape {tuple(q.shape)}")
        q = q[:, :, 0]
    if q.dim() != 3 or k.dim() != 4 or k.shape != v.shape or q.shape[:2] != k.shape[:2] or q.shape[-1] != k.shape[-1]:
        raise ValueError(f"q (B, H, D) and k, v (B, H, t, D) must all be with matching B, H, D; "
                         f"got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    check_inputs(k, k, v)
    check_inputs(q[:, :, None], q[:, :, None], q[:, :, None])
    exempt = _check_exempt(exempt)
    batch, heads, t, head_dim = k.shape
    if (selected.dim() != 3 or selected.shape[0] != batch or heads % selected.shape[1] != 0
            or selected.shape[2] < t or selected.dtype != torch.float32 or selected.device != q.device
            or selected.stride(2) != 1 or selected.stride(0) != selected.shape[1] * selected.stride(1)):
        raise ValueError(f"selected must be a (B, G, >= {t}) fp32 tensor with G dividing H, rows a fixed "
                         f"stride apart, on q's device")
    groups = selected.shape[1]
    lib = _lib.load()
    # bf16 caches are read as bf16; anything else as fp32 (exact for fp16 and fp32 values)
    dtype = _lib.DTYPE_BF16 if k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16 else _lib.DTYPE_F32
    n = batch * heads
    kdim = _kernel_dim(head_dim)
    dev = q.device
    qs = _storage(q[:, :, None], n, dtype, kdim)
    ks, kstride = _kv_storage(k, n, dtype, kdim, True)
    vs, vstride = _kv_storage(v, n, dtype, kdim, True)
    if kstride != vstride:
        ks, vs = _storage(k, n, dtype, kdim), _storage(v, n, dtype, kdim)
        kstride = t * kdim
    out = torch.empty(n, kdim, device=dev, dtype=torch.float32)
    ws_bytes = lib.sa_decode_workspace_bytes(batch, heads, t, kdim)
    ws = torch.empty(max(int(ws_bytes), 1), device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        _lib.check(lib.sa_decode(qs.data_ptr(), ks.data_ptr(), vs.data_ptr(), out.data_ptr(), selected.data_ptr(),
                                 selected.stride(1), ws.data_ptr(), ws.numel(), batch, heads, groups, t, kstride,
                                 kdim, 1.0 / math.sqrt(head_dim), dtype, exempt, _stream(dev)))
    return out[:, :head_dim].reshape(batch, heads, head_dim)


class _SelectiveAttentionFn(torch.autograd.Function):
    """Autograd wrapper (reference kernels.py:608-666): forward saves the operand tensors, the fp32
    output, row statistics and CARRY; backward runs sa_backward, head 0's selection gradient
    included."""

    @staticmethod
    def forward(ctx, q, k, v, dot_precision, block_m, block_n, num_warps, bwd_block_n, bwd_num_warps,
                bwd_num_stages, group, bwd_group, num_stages, exempt):
        check_inputs(q, k, v)
        exempt = _check_exempt(exempt)
        dtype = _resolve_precision(dot_precision, q.dtype)
        _check_blocks(block_m, block_n)
        batch, heads, seq, head_dim = q.shape
        out, rmax, rden, carry, _, (qs, ks, vs) = _forward_launch(
            q, k, v, dtype, exempt, int(group or 0), 0, 0, allow_view=False)
        ctx.save_for_backward(qs, ks, vs, out, rmax, rden, carry)
        ctx.meta = (dtype, exempt, bwd_group, head_dim, (q.dtype, k.dtype, v.dtype), batch, heads)
        result = out[..., :head_dim].reshape(batch, heads, seq, head_dim)
        return result.contiguous() if head_dim != out.shape[-1] else result

    @staticmethod
    @once_differentiable
    def backward(ctx, dout):
        qs, ks, vs, out, rmax, rden, carry = ctx.saved_tensors
        dtype, exempt, bwd_group, head_dim, dtypes, batch, heads = ctx.meta
        group = _check_bwd_group(bwd_group)
        lib = _lib.load()
        n, seq, kdim = qs.shape
        dev = qs.device
        dos = _storage(dout, n, dtype, kdim)
        # gradients leave the kernel in the input dtype when every input is stored as-is (bf16 inputs
        # on bf16 operands); otherwise in fp32, cast below (the reference's dq.to(q.dtype))
        as_bf16 = dtype == _lib.DTYPE_BF16 and all(d == torch.bfloat16 for d in dtypes)
        gdt = torch.bfloat16 if as_bf16 else torch.float32
        dq = torch.empty(qs.shape, device=dev, dtype=gdt)
        dk = torch.empty(ks.shape, device=dev, dtype=gdt)
        dv = torch.empty(vs.shape, device=dev, dtype=gdt)
        ws_bytes = lib.sa_backward_workspace_bytes(batch, heads, seq, kdim, dtype, group)
        ws = torch.empty(int(ws_bytes), device=dev, dtype=torch.uint8)
        with torch.cuda.device(dev):
            _lib.check(lib.sa_backward(
                qs.data_ptr(), ks.data_ptr(), vs.data_ptr(), out.data_ptr(), dos.data_ptr(), rmax.data_ptr(),
                rden.data_ptr(), carry.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(),
                ws.numel(), batch, heads, seq, kdim, 1.0 / math.sqrt(head_dim), dtype,
                _lib.DTYPE_BF16 if as_bf16 else _lib.DTYPE_F32, exempt, group, _stream(dev)))
        shape4 = (batch, heads, seq, head_dim)
        grads = tuple(g[..., :head_dim].reshape(shape4).to(want) for g, want in zip((dq, dk, dv), dtypes))
        return grads + (None,) * 11


class _SelectiveAttentionQKVFn(torch.autograd.Function):
    """Layer-boundary fused form of the attention call: reads q, k, v straight out of the packed
    projection (B, T, 3 * H * D) (the reference splits and transposes it, model.py:59-67), returns
    the output as (B, T, H * D) in the projection's dtype (the reference's fp32 output, cast by
    mixers.py:94, then transposed for c_proj), and writes the gradients straight into one
    (B, T, 3 * H * D) tensor (no slice gradients to assemble). The arithmetic is that of
    selective_attention: the same kernels through sa_forward_strided / sa_backward_strided."""

    @staticmethod
    def forward(ctx, qkv, heads, dot_precision, exempt):
        batch, seq, c3 = qkv.shape
        head_dim = c3 // (3 * heads)
        dtype, es = _packed_layout(qkv, heads, dot_precision)
        exempt = _check_exempt(exempt)
        lib = _lib.load()
        dev = qkv.device
        cdim = heads * head_dim
        n = batch * heads
        nb = (seq + CARRY_M - 1) // CARRY_M
        y = torch.empty(batch, seq, cdim, device=dev, dtype=qkv.dtype)
        out = torch.empty(n, seq, head_dim, device=dev, dtype=torch.float32)
        rmax = torch.empty(n, seq, device=dev, dtype=torch.float32)
        rden = torch.empty(n, seq, device=dev, dtype=torch.float32)
        carry = torch.empty(batch, nb, seq, device=dev, dtype=torch.float32)
        state = torch.empty(batch, seq, device=dev, dtype=torch.float32)
        ws = torch.empty(max(int(lib.sa_forward_workspace_bytes(batch, heads, seq, head_dim, dtype)), 1),
                         device=dev, dtype=torch.uint8)
        qkv_s = _lib.ViewStrides(seq * c3, head_dim, c3)
        y_s = _lib.ViewStrides(seq * cdim, head_dim, cdim)
        base = qkv.data_ptr()
        with torch.cuda.device(dev):
            _lib.check(lib.sa_forward_strided(
                base, qkv_s, base + cdim * es, qkv_s, base + 2 * cdim * es, qkv_s, out.data_ptr(), y.data_ptr(),
                y_s, rmax.data_ptr(), rden.data_ptr(), carry.data_ptr(), None, state.data_ptr(), state.stride(0),
                ws.data_ptr(), ws.numel(), batch, heads, seq, seq, 0, head_dim, 1.0 / math.sqrt(head_dim), dtype,
                exempt, 0, 0, 0, _stream(dev)))
        ctx.save_for_backward(qkv, out, rmax, rden, carry)
        ctx.meta = (dtype, es, exempt, heads, head_dim)
        return y

    @staticmethod
    @once_differentiable
    def backward(ctx, dy):
        qkv, out, rmax, rden, carry = ctx.saved_tensors
        dtype, es, exempt, heads, head_dim = ctx.meta
        lib = _lib.load()
        batch, seq, c3 = qkv.shape
        cdim = heads * head_dim
        dev = qkv.device
        dy = dy.to(qkv.dtype).contiguous()
        dqkv = torch.empty_like(qkv)
        ws = torch.empty(int(lib.sa_backward_workspace_bytes(batch, heads, seq, head_dim, dtype, 0)), device=dev,
                         dtype=torch.uint8)
        qkv_s = _lib.ViewStrides(seq * c3, head_dim, c3)
        dy_s = _lib.ViewStrides(seq * cdim, head_dim, cdim)
        base, gbase = qkv.data_ptr(), dqkv.data_ptr()
        with torch.cuda.device(dev):
            _lib.check(lib.sa_backward_strided(
                base, qkv_s, base + cdim * es, qkv_s, base + 2 * cdim * es, qkv_s, out.data_ptr(), dy.data_ptr(),
                dy_s, rmax.data_ptr(), rden.data_ptr(), carry.data_ptr(), gbase, qkv_s, gbase + cdim * es, qkv_s,
                gbase + 2 * cdim * es, qkv_s, ws.data_ptr(), ws.numel(), batch, heads, seq, head_dim,
                1.0 / math.sqrt(head_dim), dtype, dtype, exempt, 0, _stream(dev)))
        return dqkv, None, None, None


def _packed_layout(qkv: torch.Tensor, heads: int, dot_precision: str | None) -> tuple[int, int]:
    """(storage dtype code, element size) of a packed projection the fused form can read in place;
    ValueError otherwise."""

    if qkv.dim() != 3 or not qkv.is_cuda or qkv.shape[-1] % (3 * heads) != 0:
        raise ValueError(f"qkv must be a CUDA (B, T, 3 * heads * D) tensor; got {tuple(qkv.shape)}, heads={heads}")
    head_dim = qkv.shape[-1] // (3 * heads)
    if head_dim not in (32, 64, 128):
        raise ValueError(f"the packed form takes head_dim 32, 64 or 128; got {head_dim}")
    dtype = _resolve_precision(dot_precision, qkv.dtype)
    want = torch.bfloat16 if dtype == _lib.DTYPE_BF16 else torch.float32
    if qkv.dtype != want:
        raise ValueError(f"the packed form reads qkv in place: its dtype must be the operand dtype {want}; "
                         f"got {qkv.dtype}")
    if not qkv.is_contiguous() or qkv.data_ptr() % 16:
        raise ValueError("qkv must be contiguous and 16-byte aligned")
    if not HAS_HIP:
        _lib.load()   # raises RuntimeError with the reason
    return dtype, qkv.element_size()


def packed_supported(qkv: torch.Tensor, heads: int, dot_precision: str | None = None) -> bool:
    """True when selective_attention_qkv can read this projection in place."""

    try:
        _packed_layout(qkv, heads, dot_precision)
    except (ValueError, RuntimeError):
        return False
    return True


def selective_attention_qkv(qkv: torch.Tensor, heads: int, dot_precision: str | None = None,
                            exempt: int = 1) -> torch.Tensor:
    """Differentiable Selective Attention on a packed projection: qkv (B, T, 3 * heads * D), laid out
    as (B, T, 3, heads, D) like the reference's c_attn output (model.py:59-67), read in place; returns
    (B, T, heads * D) in qkv's dtype, the layout the output projection reads. Equal to
    selective_attention on the split heads with the output cast to qkv's dtype and merged
    (mixers.py:94, model.py:69-71). qkv's dtype must be the operand dtype (bf16, or fp32 under
    dot_precision "tf32" or "ieee"); see packed_supported."""

    return _SelectiveAttentionQKVFn.apply(qkv, int(heads), dot_precision, exempt)


def selective_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dot_precision: str | None = None,
    block_m: int | None = None,
    block_n: int = 32,
    num_warps: int = 4,
    bwd_block_n: int = 32,
    bwd_num_warps: int = 4,
    bwd_num_stages: int = 1,
    group: int | None = None,
    bwd_group: int | None = None,
    num_stages: int | None = None,
    exempt: int = 1,
) -> torch.Tensor:
    """Differentiable fused Selective Attention (reference kernels.py:669-703). q / k / v: (B, H, T, D)
    CUDA (ROCm) tensors (fp16, bf16 or fp32; D in 16, 32, 64, 128). Returns fp32 (B, H, T, D).

    T is a runtime argument of the kernels: no per-length compilation.
    """

    return _SelectiveAttentionFn.apply(q, k, v, dot_precision, block_m, block_n, num_warps,
                                       bwd_block_n, bwd_num_warps, bwd_num_stages, group, bwd_group,
                                       num_stages, exempt)
