"""CPU oracle for Selective Attention -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and
only as the checker (or the timed CPU baseline). The product path (selective_attention/) never
calls it.

A restatement, written from the operator's definition, of the reference's paper listing
(reference src/selective_attention/kernels.py:61-83; README.md:96-101; kernels.py:6-10):

    L_h[i,j] = s q_h[i].k_h[j]            s = 1/sqrt(D), causal j <= i
    S[r,j]   = relu(L_0[r,j]) for E <= j < r, else 0     (head 0 of the sequence)
    F[i,j]   = sum_{r<i} S[r,j]
    out_h    = softmax_j(L_h - F) v_h
    total[j] = sum_r S[r,j]                              (`selected_total`, kernels.py:547-549)

and of its gradient (reference docs/kernel.md:32-46). Every function works in the dtype of its
inputs (float64 for the parity checks, float32 for the timed CPU baseline).

How each function is pinned (tests/test_oracle.py):
  attention            == per-query brute-force loop (attention_loop); == SDPA when no key can be
                          selected; rows of the attention sum to 1; BOS column / diagonal untouched
  attention_loop       written per query from the definition; agrees with `attention`, which is
                          written per matrix (two formulations, a dropped term fails one of them)
  backward             analytic formulas vs torch.autograd of `attention`; autograd of `attention`
                          vs torch.autograd.gradcheck (finite differences, fp64)
  selection_totals     == column sums of the S built by attention_loop; total[:E] == 0,
                          total[T-1] == 0
  tail                 == the last rows of `attention` (chunked summation of the history)
  prefill_chunks       == `attention` (chunk state carried between calls)
  decode_steps         == `attention` (one query at a time, reference mixers.py:115-130)
  decode_step          through decode_steps (its every step); a step from an arbitrary state ==
                          the softmax written out with exp and sums
  per_head             == every head run alone as a one-head sequence (mixers.py:76-84)
No function here is "parity unpinned".
"""

from __future__ import annotations

import math

import torch


def _check_exempt(exempt: int) -> int:
    if int(exempt) != exempt or exempt < 1:
        raise ValueError(f"exempt must be an integer >= 1; got {exempt}")
    return int(exempt)


def _selectable(t_q: int, t_k: int, q_offset: int, exempt: int, device) -> torch.Tensor:
    """(t_q, t_k) bool: key j can be selected by query q_offset + r (exempt <= j < query)."""
    r = torch.arange(t_q, device=device)[:, None] + q_offset
    j = torch.arange(t_k, device=device)[None, :]
    return (j < r) & (j >= exempt)


def raw_logits(q: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
    """s q k^T, (B, H, Tq, Tk), no mask."""
    return torch.matmul(q, k.transpose(-2, -1)) * (1.0 / math.sqrt(q.shape[-1]))


def selection(q: torch.Tensor, k: torch.Tensor, exempt: int = 1, q_offset: int = 0) -> torch.Tensor:
    """S (B, Tq, Tk): head 0's relu'd logits where selectable (reference kernels.py:70-72)."""
    exempt = _check_exempt(exempt)
    l0 = raw_logits(q[:, :1], k[:, :1])[:, 0]
    mask = _selectable(q.shape[-2], k.shape[-2], q_offset, exempt, q.device)
    return torch.where(mask, torch.clamp(l0, min=0), torch.zeros((), dtype=l0.dtype))


def history(sel: torch.Tensor) -> torch.Tensor:
    """F[i,j] = sum_{r<i} S[r,j] via a strictly lower-triangular ones matrix (an independent
    formulation from the listing's roll + cumsum, kernels.py:73-75)."""
    t = sel.shape[-2]
    strict = torch.ones(t, t, dtype=sel.dtype, device=sel.device).tril(-1)
    return torch.matmul(strict, sel)


def adjusted_logits(q, k, exempt: int = 1):
    """(L - F with -inf above the diagonal, total): the listing's `selective_logits`."""
    t = q.shape[-2]
    sel = selection(q, k, exempt)
    lg = raw_logits(q, k) - history(sel)[:, None]
    causal = torch.ones(t, t, dtype=torch.bool, device=q.device).tril()
    return lg.masked_fill(~causal, float("-inf")), sel.sum(dim=-2)


def attention(q, k, v, exempt: int = 1) -> torch.Tensor:
    """out (B, H, T, D) in the input dtype (differentiable)."""
    return torch.matmul(adjusted_logits(q, k, exempt)[0].softmax(dim=-1), v)


def selection_totals(q, k, exempt: int = 1) -> torch.Tensor:
    """total (B, T): selection each key received from all queries."""
    return selection(q, k, exempt).sum(dim=-2)


def attention_loop(q, k, v, exempt: int = 1) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-query brute force from the definition: a running per-key vector is subtracted from each
    query's logits, then the query's own selection is added (reference
    tests/test_selective_kernels.py:24-40 pattern). Returns (out, total)."""
    exempt = _check_exempt(exempt)
    bsz, heads, t, d = q.shape
    out = torch.zeros(bsz, heads, t, v.shape[-1], dtype=q.dtype)
    totals = torch.zeros(bsz, t, dtype=q.dtype)
    for b in range(bsz):
        masked = torch.zeros(t, dtype=q.dtype)
        for i in range(t):
            lg = (q[b, :, i:i + 1, :] @ k[b, :, : i + 1, :].transpose(-2, -1))[:, 0, :] / math.sqrt(d)
            w = torch.softmax(lg - masked[: i + 1], dim=-1)
            out[b, :, i] = (w[:, None, :] @ v[b, :, : i + 1])[:, 0]
            sel = torch.clamp(lg[0], min=0)
            sel[: min(exempt, i + 1)] = 0
            sel[i] = 0
            masked[: i + 1] += sel
        totals[b] = masked
    return out, totals


def backward(q, k, v, dout, exempt: int = 1):
    """Analytic gradient (dq, dk, dv) of sum(out * dout), written from the chain rule
    (reference docs/kernel.md:32-46):
        z = L - F, A = softmax(z), dz = A (dout v^T - rowsum(dout * out))
        dv = A^T dout, dq = s dz k, dk = s dz^T q
        U[r,j] = sum_h sum_{i>r} dz_h[i,j];  dL_0 += -[selectable & L_0 > 0] U
    """
    s = 1.0 / math.sqrt(q.shape[-1])
    t = q.shape[-2]
    z, _ = adjusted_logits(q, k, exempt)
    a = z.softmax(dim=-1)
    out = a @ v
    dv = a.transpose(-2, -1) @ dout
    dz = a * (dout @ v.transpose(-2, -1) - (dout * out).sum(-1, keepdim=True))
    dz_sum = dz.sum(dim=1)                                          # over heads
    strict_upper = torch.ones(t, t, dtype=q.dtype).triu(1)          # [r, i] = 1 for i > r
    u = strict_upper @ dz_sum                                       # U[r, j]
    l0 = raw_logits(q[:, :1], k[:, :1])[:, 0]
    gate = _selectable(t, t, 0, _check_exempt(exempt), q.device) & (l0 > 0)
    dl = dz.clone()
    dl[:, 0] = dl[:, 0] - torch.where(gate, u, torch.zeros((), dtype=u.dtype))
    dq = s * dl @ k
    dk = s * dl.transpose(-2, -1) @ q
    return dq, dk, dv


def tail(q, k, v, tail_len: int, chunk: int = 1024, exempt: int = 1):
    """Rows [T - tail_len, T) of the output without (T x T) tensors: the history of earlier queries
    is summed chunk by chunk (reference tests/test_selective_kernels.py:310-330 form).
    Returns (rows, out_rows, total)."""
    bsz, heads, t, d = q.shape
    start = t - tail_len
    dev = q.device
    earlier = torch.zeros(bsz, t, dtype=q.dtype, device=dev)
    for a in range(0, start, chunk):
        e = min(a + chunk, start)
        earlier += selection(q[:, :, a:e], k, exempt, q_offset=a).sum(dim=1)
    sel = selection(q[:, :, start:], k, exempt, q_offset=start)
    hist = earlier[:, None, :] + torch.cumsum(sel, dim=1) - sel
    lg = raw_logits(q[:, :, start:], k) - hist[:, None]
    rows = torch.arange(start, t, device=dev)
    lg = lg.masked_fill(torch.arange(t, device=dev)[None, None, None, :] > rows[None, None, :, None], float("-inf"))
    return rows, lg.softmax(dim=-1) @ v, earlier + sel.sum(dim=1)


def prefill_chunks(q, k, v, chunk: int, exempt: int = 1):
    """The output computed chunk by chunk with the per-key selection state carried between chunks;
    returns (out, final state). Equal to `attention` and `selection_totals`."""
    bsz, heads, t, d = q.shape
    state = torch.zeros(bsz, t, dtype=q.dtype)
    outs = []
    for c0 in range(0, t, chunk):
        c1 = min(t, c0 + chunk)
        sel = selection(q[:, :, c0:c1], k[:, :, :c1], exempt, q_offset=c0)   # (B, Tc, c1)
        hist = state[:, None, :c1] + torch.cumsum(sel, dim=1) - sel
        lg = raw_logits(q[:, :, c0:c1], k[:, :, :c1]) - hist[:, None]
        rows = torch.arange(c0, c1)
        lg = lg.masked_fill(torch.arange(c1)[None, None, None, :] > rows[None, None, :, None], float("-inf"))
        outs.append(lg.softmax(dim=-1) @ v[:, :, :c1])
        state[:, :c1] += sel.sum(dim=1)
    return torch.cat(outs, dim=2), state


def decode_step(q1, k, v, state, exempt: int = 1):
    """One cached step (reference mixers.py:115-130): the query q1 (B, H, 1, D) at position t-1
    over the t cached keys, with the carried selection state (B, t) subtracted from its logits;
    returns (out (B, H, 1, D), the state with head 0's own selection of keys [E, t-1) added)."""
    t = k.shape[2]
    raw = raw_logits(q1, k)                                          # (B, H, 1, t)
    out = torch.softmax(raw - state[:, None, None, :t], dim=-1) @ v
    own = torch.clamp(raw[:, 0, 0], min=0)
    own[:, :exempt] = 0
    own[:, t - 1] = 0
    new_state = state.clone()
    new_state[:, :t] += own
    return out, new_state


def decode_steps(q, k, v, prompt: int, exempt: int = 1):
    """Rows [prompt, T) computed one query at a time (decode_step) from the selection state after
    the prompt (reference mixers.py:105-130). Returns (out_rows, final state)."""
    _, state = prefill_chunks(q[:, :, :prompt], k[:, :, :prompt], v[:, :, :prompt], prompt, exempt)
    bsz, heads, t, d = q.shape
    state = torch.cat([state, torch.zeros(bsz, t - prompt, dtype=q.dtype)], dim=1)
    outs = []
    for i in range(prompt, t):
        out, state = decode_step(q[:, :, i:i + 1], k[:, :, : i + 1], v[:, :, : i + 1], state, exempt)
        outs.append(out)
    return torch.cat(outs, dim=2), state


def per_head(q, k, v, exempt: int = 1) -> torch.Tensor:
    """Every head selects for itself: each head as its own one-head sequence (mixers.py:76-84)."""
    bsz, heads, t, d = q.shape
    r = lambda x: x.reshape(bsz * heads, 1, t, x.shape[-1])
    return attention(r(q), r(k), r(v), exempt).reshape(bsz, heads, t, v.shape[-1])
