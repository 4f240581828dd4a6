"""Selective Attention on MI355X: the reference's operator API over hand-written gfx950 HIP kernels.

The operator (Leviathan, Kalman, Matias, "Selective Attention Improves Transformer", ICLR 2025) is
causal softmax attention whose logits lose a history term. Head 0 of a sequence is the selector:
for a query r, its positive scaled logit on an earlier key j (j past the first `exempt` positions)
is how much r "selects" j. F[i, j] adds up the selection key j received from the queries before i,
and every head attends with softmax(s q.k - F) over keys j <= i (s = 1 / sqrt(head_dim)).

This module keeps the names, keyword arguments and error messages of the reference's
`selective_attention.kernels` (reference src/selective_attention/kernels.py:61-83, 427-703) so
callers switch by import path. The work runs in libsa_hip.so (include/sa.h):

    selection   column sums of head 0's selection per 32-query block, then an exclusive running
                sum: CARRY (B, ceil(T/32), T) fp32, the reference's checkpoint layout, plus totals
    forward     query-parallel online softmax of L_h - F on bf16 (or fp32) MFMA
    backward    a key-side kernel (dK, dV, head 0's selection gradient) and a query-side kernel (dQ)

Each C-ABI call is a `torch.library` custom op (namespace `selective_attention`: forward, backward,
qkv_forward, qkv_backward) with a fake (meta) implementation, so `torch.compile` traces through
`selective_attention` / `selective_attention_qkv` without a graph break; the autograd functions are
built on those ops.

`dot_precision` picks the MFMA operand type: "bf16" (default for bf16 inputs) runs bf16 operands
with fp32 accumulation; "tf32" (default otherwise) and "ieee" both run fp32 operands on fp32 MFMA,
since gfx950 has no TF32 datapath (so "tf32" is exact fp32 here). fp16 inputs are converted to the
operand type; outputs are fp32 as in the reference, gradients come back in the input dtypes.

Tile and launch kwargs of the reference (block_m, block_n, num_warps, num_stages, bwd_block_n,
bwd_num_warps, bwd_num_stages) are accepted and validated as the reference does, but do not change
the launch: the HIP kernels use 32 x 32 MFMA tiles and 256-thread workgroups. `group` (forward) and
`bwd_group` (backward) set the heads per wavefront, within what the kernels instantiate (results do
not depend on them beyond fp32 summation order).

On CUDA (ROCm) tensors the HIP library must load, or these functions raise RuntimeError: there is
no silent fallback. `selective_logits` / `selective_attention_reference` are the plain torch
listing, exported as in the reference.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import Tensor

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

def selective_logits(q: Tensor, k: Tensor, exempt: int = 1) -> tuple[Tensor, Tensor]:
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


def selective_attention_reference(q: Tensor, k: Tensor, v: Tensor, exempt: int = 1) -> Tensor:
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


def check_inputs(q: Tensor, k: Tensor, v: Tensor) -> None:
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


def supported(q: Tensor, k: Tensor | None = None, v: Tensor | None = None) -> bool:
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


def _storage_dtype(code: int) -> torch.dtype:
    return torch.bfloat16 if code == _lib.DTYPE_BF16 else torch.float32


def _code_of(t: Tensor) -> int:
    return _lib.DTYPE_BF16 if t.dtype == torch.bfloat16 else _lib.DTYPE_F32


def _storage(t: Tensor, code: int, kdim: int) -> Tensor:
    """(..., T, D) -> contiguous (..., T, kdim) in the operand storage dtype."""

    x = t.to(_storage_dtype(code))
    if kdim != t.shape[-1]:
        x = F.pad(x, (0, kdim - t.shape[-1]))
    return x.contiguous()


def _kv_storage(t: Tensor, code: int, kdim: int) -> tuple[Tensor, int]:
    """(B, H, T, D) keys or values for sa_forward, and the element stride between heads. A view whose
    heads sit a fixed stride apart with contiguous (T, D) rows inside each head (a slice of a
    preallocated cache) is passed as is; anything else becomes contiguous first."""

    batch, heads, seq, head_dim = t.shape
    if t.dtype == _storage_dtype(code) and head_dim == kdim and t.stride(3) == 1 and t.stride(2) == head_dim:
        # flattened row r = b * heads + h must start at r * hs
        if heads > 1:
            hs = t.stride(1)
            rows_ok = batch == 1 or t.stride(0) == heads * hs
        else:
            hs = t.stride(0) if batch > 1 else seq * head_dim
            rows_ok = True
        if rows_ok and hs >= seq * head_dim and hs % 8 == 0 and t.data_ptr() % 16 == 0:
            return t, hs
    return _storage(t, code, kdim), seq * kdim


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _launch_forward(qs: Tensor, ks: Tensor, vs: Tensor, kstride: int, scale: float, exempt: int, group: int,
                    damp_mode: int, train_len: int, state_in: Tensor | None = None, q_offset: int = 0,
                    state: Tensor | None = None):
    """sa_forward on storage tensors: qs (B, H, Tq, Dk) contiguous; ks, vs (B, H, Tk, Dk) with heads
    `kstride` elements apart. Returns out (B, H, Tq, Dk) fp32, rmax, rden (B, H, Tq), carry
    (B, ceil(Tq/32), Tk) and the per-key state (B, >= Tk)."""

    lib = _lib.load()
    batch, heads, tq, kdim = qs.shape
    tk = ks.shape[-2]
    dev = qs.device
    code = _code_of(qs)
    nb = (tq + CARRY_M - 1) // CARRY_M
    out = torch.empty(batch, heads, tq, kdim, device=dev, dtype=torch.float32)
    rmax = torch.empty(batch, heads, tq, device=dev, dtype=torch.float32)
    rden = torch.empty(batch, heads, tq, device=dev, dtype=torch.float32)
    carry = torch.empty(batch, nb, tk, device=dev, dtype=torch.float32)
    if state is None:
        state = torch.empty(batch, tk, device=dev, dtype=torch.float32)
    ws = torch.empty(max(int(lib.sa_forward_workspace_bytes(batch, heads, tk, kdim, code, group)), 1), device=dev,
                     dtype=torch.uint8)
    with torch.cuda.device(dev):
        _lib.check(lib.sa_forward(
            qs.data_ptr(), ks.data_ptr(), vs.data_ptr(), out.data_ptr(), rmax.data_ptr(), rden.data_ptr(),
            carry.data_ptr(), None if state_in is None else state_in.data_ptr(), state.data_ptr(),
            state.stride(0), ws.data_ptr(), ws.numel(), batch, heads, tq, tk, q_offset, kstride, kdim, scale, code,
            exempt, group, damp_mode, train_len, _stream(dev)))
    return out, rmax, rden, carry, state


# -- the C-ABI calls as custom ops ------------------------------------------------------------------

@torch.library.custom_op("selective_attention::forward", mutates_args=(), device_types="cuda")
def _forward_op(q: Tensor, k: Tensor, v: Tensor, scale: float, exempt: int, group: int, damp_mode: int,
                train_len: int) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """sa_forward on contiguous (B, H, T, Dk) storage tensors (bf16 or fp32): out (B, H, T, Dk) fp32,
    rmax, rden (B, H, T), carry (B, ceil(T/32), T), selected_total (B, T)."""
    return _launch_forward(q, k, v, k.shape[-2] * k.shape[-1], scale, exempt, group, damp_mode, train_len)


@_forward_op.register_fake
def _forward_fake(q, k, v, scale, exempt, group, damp_mode, train_len):
    batch, heads, seq, kdim = q.shape
    nb = (seq + CARRY_M - 1) // CARRY_M
    f32 = dict(dtype=torch.float32)
    return (q.new_empty((batch, heads, seq, kdim), **f32), q.new_empty((batch, heads, seq), **f32),
            q.new_empty((batch, heads, seq), **f32), q.new_empty((batch, nb, seq), **f32),
            q.new_empty((batch, seq), **f32))


@torch.library.custom_op("selective_attention::backward", mutates_args=(), device_types="cuda")
def _backward_op(q: Tensor, k: Tensor, v: Tensor, out: Tensor, dout: Tensor, rmax: Tensor, rden: Tensor,
                 carry: Tensor, scale: float, exempt: int, group: int,
                 grad_bf16: bool) -> tuple[Tensor, Tensor, Tensor]:
    """sa_backward: dq, dk, dv (B, H, T, Dk) in bf16 (grad_bf16) or fp32, from the storage tensors,
    the forward's fp32 output, row statistics and CARRY, and dout in the storage dtype."""
    lib = _lib.load()
    batch, heads, seq, kdim = q.shape
    dev = q.device
    code = _code_of(q)
    gdt = torch.bfloat16 if grad_bf16 else torch.float32
    dq, dk, dv = (torch.empty(q.shape, device=dev, dtype=gdt) for _ in range(3))
    ws = torch.empty(int(lib.sa_backward_workspace_bytes(batch, heads, seq, kdim, code, group)), device=dev,
                     dtype=torch.uint8)
    with torch.cuda.device(dev):
        _lib.check(lib.sa_backward(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), dout.data_ptr(), rmax.data_ptr(),
            rden.data_ptr(), carry.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(),
            ws.numel(), batch, heads, seq, kdim, scale, code, _lib.DTYPE_BF16 if grad_bf16 else _lib.DTYPE_F32,
            exempt, group, _stream(dev)))
    return dq, dk, dv


@_backward_op.register_fake
def _backward_fake(q, k, v, out, dout, rmax, rden, carry, scale, exempt, group, grad_bf16):
    gdt = torch.bfloat16 if grad_bf16 else torch.float32
    return tuple(q.new_empty(q.shape, dtype=gdt) for _ in range(3))


def _packed_strides(batch: int, seq: int, heads: int, head_dim: int):
    """View strides of q, k, v (and their gradients) in a packed (B, T, 3 * H * D) projection and of
    the (B, T, H * D) output."""
    c3, cdim = 3 * heads * head_dim, heads * head_dim
    return _lib.ViewStrides(seq * c3, head_dim, c3), _lib.ViewStrides(seq * cdim, head_dim, cdim)


@torch.library.custom_op("selective_attention::qkv_forward", mutates_args=(), device_types="cuda")
def _qkv_forward_op(qkv: Tensor, heads: int, exempt: int) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """sa_forward_strided on a packed (B, T, 3 * H * D) projection read in place: the output y
    (B, T, H * D) in qkv's dtype, and the fp32 output (B, H, T, D), rmax, rden, carry saved for the
    backward."""
    lib = _lib.load()
    batch, seq, c3 = qkv.shape
    head_dim = c3 // (3 * heads)
    cdim = heads * head_dim
    dev = qkv.device
    code, es = _code_of(qkv), qkv.element_size()
    y = torch.empty(batch, seq, cdim, device=dev, dtype=qkv.dtype)
    out = torch.empty(batch, heads, seq, head_dim, device=dev, dtype=torch.float32)
    rmax = torch.empty(batch, heads, seq, device=dev, dtype=torch.float32)
    rden = torch.empty(batch, heads, seq, device=dev, dtype=torch.float32)
    carry = torch.empty(batch, (seq + CARRY_M - 1) // CARRY_M, seq, device=dev, dtype=torch.float32)
    state = torch.empty(batch, seq, device=dev, dtype=torch.float32)
    ws = torch.empty(max(int(lib.sa_forward_workspace_bytes(batch, heads, seq, head_dim, code, 0)), 1), device=dev,
                     dtype=torch.uint8)
    qkv_s, y_s = _packed_strides(batch, seq, heads, head_dim)
    base = qkv.data_ptr()
    with torch.cuda.device(dev):
        _lib.check(lib.sa_forward_strided(
            base, qkv_s, base + cdim * es, qkv_s, base + 2 * cdim * es, qkv_s, out.data_ptr(), y.data_ptr(), y_s,
            rmax.data_ptr(), rden.data_ptr(), carry.data_ptr(), None, state.data_ptr(), state.stride(0),
            ws.data_ptr(), ws.numel(), batch, heads, seq, seq, 0, head_dim, 1.0 / math.sqrt(head_dim), code,
            exempt, 0, 0, 0, _stream(dev)))
    return y, out, rmax, rden, carry


@_qkv_forward_op.register_fake
def _qkv_forward_fake(qkv, heads, exempt):
    batch, seq, c3 = qkv.shape
    head_dim = c3 // (3 * heads)
    f32 = dict(dtype=torch.float32)
    return (qkv.new_empty((batch, seq, heads * head_dim)), qkv.new_empty((batch, heads, seq, head_dim), **f32),
            qkv.new_empty((batch, heads, seq), **f32), qkv.new_empty((batch, heads, seq), **f32),
            qkv.new_empty((batch, (seq + CARRY_M - 1) // CARRY_M, seq), **f32))


@torch.library.custom_op("selective_attention::qkv_backward", mutates_args=(), device_types="cuda")
def _qkv_backward_op(qkv: Tensor, dy: Tensor, out: Tensor, rmax: Tensor, rden: Tensor, carry: Tensor, heads: int,
                     exempt: int) -> Tensor:
    """sa_backward_strided for the packed form: the gradient of qkv as one (B, T, 3 * H * D) tensor,
    from dy (B, T, H * D) in qkv's dtype."""
    lib = _lib.load()
    batch, seq, c3 = qkv.shape
    head_dim = c3 // (3 * heads)
    cdim = heads * head_dim
    dev = qkv.device
    code, es = _code_of(qkv), qkv.element_size()
    dqkv = torch.empty_like(qkv)
    ws = torch.empty(int(lib.sa_backward_workspace_bytes(batch, heads, seq, head_dim, code, 0)), device=dev,
                     dtype=torch.uint8)
    qkv_s, dy_s = _packed_strides(batch, seq, heads, head_dim)
    base, gbase = qkv.data_ptr(), dqkv.data_ptr()
    with torch.cuda.device(dev):
        _lib.check(lib.sa_backward_strided(
            base, qkv_s, base + cdim * es, qkv_s, base + 2 * cdim * es, qkv_s, out.data_ptr(), dy.data_ptr(), dy_s,
            rmax.data_ptr(), rden.data_ptr(), carry.data_ptr(), gbase, qkv_s, gbase + cdim * es, qkv_s,
            gbase + 2 * cdim * es, qkv_s, ws.data_ptr(), ws.numel(), batch, heads, seq, head_dim,
            1.0 / math.sqrt(head_dim), code, code, exempt, 0, _stream(dev)))
    return dqkv


@_qkv_backward_op.register_fake
def _qkv_backward_fake(qkv, dy, out, rmax, rden, carry, heads, exempt):
    return torch.empty_like(qkv)


# -- the operator API ---------------------------------------------------------------------------------

def selective_attention_forward(
    q: Tensor,
    k: Tensor,
    v: Tensor,
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
    code = _resolve_precision(dot_precision, q.dtype)
    _check_blocks(block_m, block_n)
    damp_mode = _damp_mode(damp, train_len)
    head_dim = q.shape[-1]
    kdim = _kernel_dim(head_dim)
    qs, ks, vs = (_storage(t, code, kdim) for t in (q, k, v))
    out, rmax, rden, carry, total = _forward_op(qs, ks, vs, 1.0 / math.sqrt(head_dim), exempt, int(group or 0),
                                                damp_mode, int(train_len))
    result = out[..., :head_dim].contiguous() if kdim != head_dim else out
    if return_aux:
        n = q.shape[0] * q.shape[1]
        return result, dict(rmax=rmax.reshape(n, -1), rden=rden.reshape(n, -1), carry=carry, selected_total=total)
    return result


def selective_attention_prefill(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    state: Tensor,
    q_offset: int,
    dot_precision: str | None = None,
    exempt: int = 1,
    group: int | None = None,
) -> Tensor:
    """One chunk of a chunked prefill (no reference counterpart: the reference runs long inputs as one
    forward with a T^2/8-byte CARRY, kernels.py:38-40).

    q: (B, H, Tc, D), the queries at absolute positions [q_offset, q_offset + Tc). k, v:
    (B, H, q_offset + Tc, D), every key and value so far (a slice of a preallocated cache is read in
    place). state: (B, L) fp32, L >= q_offset + Tc, holding for every key j < q_offset the selection
    received from all queries before q_offset; it is updated in place to cover the queries of this
    chunk too (entries >= q_offset are overwritten). Returns fp32 (B, H, Tc, D), equal to rows
    [q_offset, q_offset + Tc) of the single-shot forward.
    """

    if q.dim() != 4 or k.shape != v.shape or q.shape[:2] != k.shape[:2] or q.shape[-1] != k.shape[-1]:
        raise ValueError(f"q (B, H, Tc, D) and k, v (B, H, Tk, D) must all be 4-D with matching B, H, D; "
                         f"got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    check_inputs(q, q, q)
    check_inputs(k, k, v)
    exempt = _check_exempt(exempt)
    code = _resolve_precision(dot_precision, q.dtype)
    batch, heads, tc, head_dim = q.shape
    tk = k.shape[-2]
    if q_offset < 0 or q_offset + tc != tk:
        raise ValueError(f"k and v must hold q_offset + Tc = {q_offset + tc} positions; got {tk}")
    if (state.dim() != 2 or state.shape[0] != batch or state.shape[1] < tk or state.dtype != torch.float32
            or state.device != q.device or state.stride(1) != 1):
        raise ValueError(f"state must be a (B, >= {tk}) fp32 tensor with unit column stride on q's device")
    kdim = _kernel_dim(head_dim)
    qs = _storage(q, code, kdim)
    ks, kstride = _kv_storage(k, code, kdim)
    vs, vstride = _kv_storage(v, code, kdim)
    if kstride != vstride:   # one stride serves both: contiguous copies
        ks, vs = _storage(k, code, kdim), _storage(v, code, kdim)
        kstride = tk * kdim
    out, *_ = _launch_forward(qs, ks, vs, kstride, 1.0 / math.sqrt(head_dim), exempt, int(group or 0), 0, 0,
                              state_in=state if q_offset > 0 else None, q_offset=int(q_offset), state=state)
    return out[..., :head_dim]


def selective_attention_decode(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    selected: Tensor,
    exempt: int = 1,
) -> Tensor:
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
    # q's own checks (its head dim equals k's, checked above), without building the 4-D views
    # check_inputs takes: a decode step is host-bound at short caches, so its checks stay cheap
    if not (q.is_cuda and q.device == k.device):
        raise ValueError("q, k, v must be CUDA (ROCm) tensors on one device")
    if q.dtype not in DTYPES:
        raise ValueError(f"dtype must be float16, bfloat16 or float32; got {q.dtype}, {k.dtype}, {v.dtype}")
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
    code = _lib.DTYPE_BF16 if k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16 else _lib.DTYPE_F32
    kdim = _kernel_dim(head_dim)
    dev = q.device
    qs = _storage(q, code, kdim)
    ks, kstride = _kv_storage(k, code, kdim)
    vs, vstride = _kv_storage(v, code, kdim)
    if kstride != vstride:
        ks, vs = _storage(k, code, kdim), _storage(v, code, kdim)
        kstride = t * kdim
    out = torch.empty(batch, heads, kdim, device=dev, dtype=torch.float32)
    ws = torch.empty(max(int(lib.sa_decode_workspace_bytes(batch, heads, t, kdim)), 1), device=dev, dtype=torch.uint8)
    def launch():
        _lib.check(lib.sa_decode(qs.data_ptr(), ks.data_ptr(), vs.data_ptr(), out.data_ptr(), selected.data_ptr(),
                                 selected.stride(1), ws.data_ptr(), ws.numel(), batch, heads, groups, t, kstride,
                                 kdim, 1.0 / math.sqrt(head_dim), code, exempt, _stream(dev)))

    # (a device guard only when q's device is not already the current one: it costs a few us a step)
    if dev.index == torch.cuda.current_device():
        launch()
    else:
        with torch.cuda.device(dev):
            launch()
    return out[..., :head_dim]


class _SelectiveAttentionFn(torch.autograd.Function):
    """Autograd wrapper (reference kernels.py:608-666) over the forward / backward custom ops: forward
    saves the operand tensors, the fp32 output, row statistics and CARRY; backward runs the
    backward op, head 0's selection gradient included."""

    @staticmethod
    def forward(ctx, q, k, v, dot_precision, block_m, block_n, num_warps, bwd_block_n, bwd_num_warps,
                bwd_num_stages, group, bwd_group, num_stages, exempt):
        check_inputs(q, k, v)
        exempt = _check_exempt(exempt)
        code = _resolve_precision(dot_precision, q.dtype)
        _check_blocks(block_m, block_n)
        head_dim = q.shape[-1]
        kdim = _kernel_dim(head_dim)
        qs, ks, vs = (_storage(t, code, kdim) for t in (q, k, v))
        out, rmax, rden, carry, _ = _forward_op(qs, ks, vs, 1.0 / math.sqrt(head_dim), exempt, int(group or 0),
                                                0, 0)
        ctx.save_for_backward(qs, ks, vs, out, rmax, rden, carry)
        ctx.exempt, ctx.bwd_group, ctx.head_dim = exempt, bwd_group, head_dim
        ctx.in_dtypes = (q.dtype, k.dtype, v.dtype)
        return out[..., :head_dim].contiguous() if kdim != head_dim else out

    @staticmethod
    def backward(ctx, dout):
        qs, ks, vs, out, rmax, rden, carry = ctx.saved_tensors
        group = _check_bwd_group(ctx.bwd_group)
        head_dim, kdim = ctx.head_dim, qs.shape[-1]
        dos = _storage(dout, _code_of(qs), kdim)
        # gradients leave the kernel in the input dtype when every input is stored as-is (bf16 inputs
        # on bf16 operands); otherwise in fp32, cast below (the reference's dq.to(q.dtype))
        as_bf16 = qs.dtype == torch.bfloat16 and all(d == torch.bfloat16 for d in ctx.in_dtypes)
        grads = _backward_op(qs, ks, vs, out, dos, rmax, rden, carry, 1.0 / math.sqrt(head_dim), ctx.exempt,
                             group, as_bf16)
        grads = tuple(g[..., :head_dim].to(want) for g, want in zip(grads, ctx.in_dtypes))
        return grads + (None,) * 11


class _SelectiveAttentionQKVFn(torch.autograd.Function):
    """Layer-boundary fused form of the attention call: reads q, k, v straight out of the packed
    projection (B, T, 3 * H * D) (the reference splits and transposes it, model.py:59-67), returns
    the output as (B, T, H * D) in the projection's dtype (the reference's fp32 output, cast by
    mixers.py:94, then transposed for c_proj), and writes the gradients straight into one
    (B, T, 3 * H * D) tensor (no slice gradients to assemble). The arithmetic is that of
    selective_attention: the same kernels, through the qkv_forward / qkv_backward ops."""

    @staticmethod
    def forward(ctx, qkv, heads, dot_precision, exempt):
        _packed_layout(qkv, heads, dot_precision)
        exempt = _check_exempt(exempt)
        y, out, rmax, rden, carry = _qkv_forward_op(qkv, heads, exempt)
        ctx.save_for_backward(qkv, out, rmax, rden, carry)
        ctx.heads, ctx.exempt = heads, exempt
        return y

    @staticmethod
    def backward(ctx, dy):
        qkv, out, rmax, rden, carry = ctx.saved_tensors
        dqkv = _qkv_backward_op(qkv, dy.to(qkv.dtype).contiguous(), out, rmax, rden, carry, ctx.heads, ctx.exempt)
        return dqkv, None, None, None


def _packed_rows_fit(seq: int, row: int, elem_size: int) -> bool:
    """The kernels address one head's rows (seq + 64 with the transposed copies' padding) with 32-bit
    byte offsets: at a row stride of `row` elements they must span less than 2 GiB (the C ABI's
    own check, rows_fit in csrc/sa_host.h)."""
    return (seq + 64) * row * elem_size < 2 ** 31


def _packed_layout(qkv: Tensor, heads: int, dot_precision: str | None) -> int:
    """The storage dtype code of a packed projection the fused form can read in place; ValueError
    otherwise."""

    if qkv.dim() != 3 or not qkv.is_cuda or qkv.shape[-1] % (3 * heads) != 0:
        raise ValueError(f"qkv must be a CUDA (B, T, 3 * heads * D) tensor; got {tuple(qkv.shape)}, heads={heads}")
    head_dim = qkv.shape[-1] // (3 * heads)
    if head_dim not in (32, 64, 128):
        raise ValueError(f"the packed form takes head_dim 32, 64 or 128; got {head_dim}")
    code = _resolve_precision(dot_precision, qkv.dtype)
    want = _storage_dtype(code)
    if qkv.dtype != want:
        raise ValueError(f"the packed form reads qkv in place: its dtype must be the operand dtype {want}; "
                         f"got {qkv.dtype}")
    # (a traced call sees no storage; the C ABI checks the alignment of the real tensor)
    if not qkv.is_contiguous() or (not torch.compiler.is_compiling() and qkv.data_ptr() % 16):
        raise ValueError("qkv must be contiguous and 16-byte aligned")
    if not _packed_rows_fit(qkv.shape[1], qkv.shape[-1], qkv.element_size()):
        raise ValueError("the packed form addresses one head's rows below 2 GiB at the packed row stride; "
                         f"T={qkv.shape[1]} with rows of {qkv.shape[-1]} elements is past it")
    if not HAS_HIP:
        _lib.load()   # raises RuntimeError with the reason
    return code


def packed_supported(qkv: Tensor, heads: int, dot_precision: str | None = None) -> bool:
    """True when selective_attention_qkv can read this projection in place."""

    try:
        _packed_layout(qkv, heads, dot_precision)
    except (ValueError, RuntimeError):
        return False
    return True


def selective_attention_qkv(qkv: Tensor, heads: int, dot_precision: str | None = None, exempt: int = 1) -> Tensor:
    """Differentiable Selective Attention on a packed projection: qkv (B, T, 3 * heads * D), laid out
    as (B, T, 3, heads, D) like the reference's c_attn output (model.py:59-67), read in place; returns
    (B, T, heads * D) in qkv's dtype, the layout the output projection reads. Equal to
    selective_attention on the split heads with the output cast to qkv's dtype and merged
    (mixers.py:94, model.py:69-71). qkv's dtype must be the operand dtype (bf16, or fp32 under
    dot_precision "tf32" or "ieee"); see packed_supported."""

    return _SelectiveAttentionQKVFn.apply(qkv, int(heads), dot_precision, exempt)


def selective_attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
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
) -> Tensor:
    """Differentiable fused Selective Attention (reference kernels.py:669-703). q / k / v: (B, H, T, D)
    CUDA (ROCm) tensors (fp16, bf16 or fp32; D in 16, 32, 64, 128). Returns fp32 (B, H, T, D).

    T is a runtime argument of the kernels: no per-length compilation.
    """

    return _SelectiveAttentionFn.apply(q, k, v, dot_precision, block_m, block_n, num_warps,
                                       bwd_block_n, bwd_num_warps, bwd_num_stages, group, bwd_group,
                                       num_stages, exempt)
