"""Measurements of the operator inside a model, for BASELINE's configurations beyond the single-layer
fwd+bwd (bench.py measures that one):

    C3  train_step_rate    one training step of the 24-layer decoder at 1 x 16384 tokens, bf16
                           autocast, fused AdamW (reference train.py:624-650, runtime.py:610-638)
    C4  prefill_rate       forward-only prefill of 131072 tokens in chunks of 16384, every layer
                           carrying its K/V and per-key selection state between chunks
    C5  perhead_rate       per-head selection fwd+bwd at B=2, H=16, T=32768, D=64 with k scaled by 2
                           on a random 10% of key positions

Synthetic inputs only: token ids uniform over the GPT-2 vocabulary with <BOS> (50256) first, the
reference's window rule input = [bos] + window[:-1], targets = window (data.py:136-139);
random-init weights. Times are HIP events around whole steps after warm-up.

    python -m selective_attention.harness c3 [--geometry d768|d1024] [--steps K] [--warmup W]
    python -m selective_attention.harness c4 [--tokens 131072] [--chunk 16384]
    python -m selective_attention.harness c5
    python -m selective_attention.harness decode [--tokens 131072]   (one decode step's HBM rate)
    python -m selective_attention.harness copy      (reference copy for rocprofv3 byte counters)
"""

from __future__ import annotations

import argparse
import json
import math
import sys

import torch

from . import _lib, kernels
from .model import ModelConfig, SelectiveLM

GPT2_VOCAB = 50257
BOS = 50256
GEOMETRIES = {
    "d768": dict(d_model=768, n_heads=12),     # the reference's 209M model (configs/scale_16384/*.yaml)
    "d1024": dict(d_model=1024, n_heads=16),   # BASELINE's literal geometry (353.5M parameters)
}
PEAK_BF16_TFLOPS = 2500.0


def synthetic_batch(batch: int, seq: int, device, seed: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """(input ids, targets): a uniform random window with <BOS> prepended to the inputs."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    window = torch.randint(0, GPT2_VOCAB, (batch, seq), generator=g)
    idx = torch.cat([torch.full_like(window[:, :1], BOS), window[:, :-1]], dim=1)
    return idx.to(device), window.to(device)


def _timed(fn, steps: int, warmup: int) -> float:
    """Milliseconds per call of fn(), HIP events around `steps` calls after `warmup` calls."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def model_flop_per_token(cfg: ModelConfig, seq: int) -> float:
    """Training FLOP per token: 6 N for the matrix products (every parameter, the tied output head
    included: its product is real work even though the embedding lookup is not) + the attention
    products, 7 H D T per layer under the FlashAttention convention (causal pairs T^2/2 counted
    once, backward 2.5 x forward)."""
    with torch.device("meta"):
        n = SelectiveLM(cfg).num_parameters()
    hd = cfg.d_model // cfg.n_heads
    return 6.0 * n + cfg.n_layers * 7.0 * cfg.n_heads * hd * seq


def train_step_rate(geometry: str = "d768", steps: int = 10, warmup: int = 3, seq: int = 16384, batch: int = 1,
                    layers: int = 24) -> dict:
    """C3: tokens per second of full training steps (forward, backward, grad clip, fused AdamW)."""
    dev = torch.device("cuda")
    cfg = ModelConfig(n_layers=layers, context_length=seq, **GEOMETRIES[geometry])
    torch.manual_seed(0)
    model = SelectiveLM(cfg).to(dev).train()
    opt = torch.optim.AdamW(model.parameters(), lr=6e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, fused=True)
    idx, targets = synthetic_batch(batch, seq, dev)
    losses = []

    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            _, loss = model(idx, targets)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
        opt.step()
        opt.zero_grad(set_to_none=True)
        losses.append(loss.detach())

    torch.cuda.reset_peak_memory_stats()
    ms = _timed(step, steps, warmup)
    final = float(losses[-1])
    if not math.isfinite(final):
        raise RuntimeError(f"non-finite training loss {final}")
    # the attention kernels' share of a step, from their own HIP events over one more step
    per_step = kernel_times(step, 1, per_call=True)
    attn_ms = sum(per_step.values())
    tokens = batch * seq
    flop = model_flop_per_token(cfg, seq) * tokens
    return {"config": f"C3 train step, {geometry} ({model.num_parameters()} params), {layers} layers, "
                      f"{batch}x{seq} tokens, bf16 autocast, fused AdamW, eager",
            "tokens_per_s": tokens / (ms * 1e-3), "ms_per_step": ms, "model_tflops": flop / (ms * 1e-3) / 1e12,
            "attention_kernel_ms": attn_ms, "attention_share": attn_ms / ms,
            "per_layer_attention_ms": {name: t / layers for name, t in per_step.items()},
            "loss": final, "peak_mem_gib": torch.cuda.max_memory_allocated() / 2**30, "steps": steps,
            "warmup": warmup}


def prefill_rate(tokens: int = 131072, chunk: int = 16384, geometry: str = "d1024", layers: int = 24,
                 reps: int = 1, warmup: int = 1) -> dict:
    """C4: tokens per second of a chunked prefill (forward only, bf16 weights)."""
    dev = torch.device("cuda")
    cfg = ModelConfig(n_layers=layers, context_length=tokens, **GEOMETRIES[geometry])
    torch.manual_seed(0)
    model = SelectiveLM(cfg).to(dev, torch.bfloat16).eval()
    idx, _ = synthetic_batch(1, tokens, dev, seed=1)

    def run():
        with torch.no_grad():
            model.prefill_chunked(idx, chunk)

    torch.cuda.reset_peak_memory_stats()
    ms = _timed(run, reps, warmup)
    per_prefill = kernel_times(run, 1, per_call=True)
    attn_ms = per_prefill["forward"] + per_prefill["selection"]
    hd = cfg.d_model // cfg.n_heads
    attn_flop = layers * 2.0 * cfg.n_heads * hd * tokens * tokens
    return {"config": f"C4 prefill, {geometry}, {layers} layers, {tokens} tokens in chunks of {chunk}, bf16",
            "tokens_per_s": tokens / (ms * 1e-3), "ms": ms,
            "attention_kernel_ms": attn_ms, "attention_share": attn_ms / ms,
            "attention_tflops": attn_flop / (attn_ms * 1e-3) / 1e12,
            "attention_frac_of_peak": attn_flop / (attn_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
            "per_layer_chunk_forward_ms": per_prefill["forward"] / (layers * ((tokens + chunk - 1) // chunk)),
            "peak_mem_gib": torch.cuda.max_memory_allocated() / 2**30}


def perhead_rate(batch: int = 2, heads: int = 16, seq: int = 32768, head_dim: int = 64, steps: int = 5,
                 warmup: int = 2) -> dict:
    """C5: per-head selection fwd+bwd TFLOP/s; each head is its own one-head sequence, keys of a
    random 10% of positions scaled by 2."""
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(5)
    q, k, v, do = (torch.randn(batch, heads, seq, head_dim, device=dev, generator=g) for _ in range(4))
    boost = torch.rand(batch, heads, seq, 1, device=dev, generator=g) < 0.1
    k = torch.where(boost, 2.0 * k, k)
    r = lambda t: t.reshape(batch * heads, 1, seq, head_dim)
    qq, kk, vv = (r(t).bfloat16().requires_grad_(True) for t in (q, k, v))
    dd = r(do)

    def step():
        out = kernels.selective_attention(qq, kk, vv)
        torch.autograd.grad(out, (qq, kk, vv), dd)

    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    ms = _timed(step, steps, warmup)
    peak = torch.cuda.max_memory_allocated() / 2**30
    kernel_ms = kernel_times(step, steps)
    unit = batch * heads * head_dim * seq * seq   # one causal product over all heads
    flop = 7.0 * unit
    tf = flop / (ms * 1e-3) / 1e12
    dominant = max(KERNEL_PRODUCTS, key=lambda name: kernel_ms[name])
    achieved = KERNEL_PRODUCTS[dominant] * unit / (kernel_ms[dominant] * 1e-3) / 1e12
    return {"config": f"C5 per-head fwd+bwd, B={batch} H={heads} T={seq} D={head_dim} bf16, k x2 on 10% of keys",
            "ms_per_step": ms, "tflops": tf, "frac_of_peak": tf / PEAK_BF16_TFLOPS,
            "kernel_ms": kernel_ms, "peak_mem_gib": peak,
            "roofline": {"bound": "mfma", "kernel": f"{dominant} ({KERNEL_PRODUCTS[dominant]:.0f}*B*H*D*T^2 FLOP)",
                         "achieved": achieved, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": achieved / PEAK_BF16_TFLOPS}}


# The reference's published one-layer figures (results/bench/layer_fwd_bwd_v2.json:26-93, op
# "selective", B=2 H=12 D=64 bf16, 20 reps on an NVIDIA RTX PRO 6000 Blackwell): seq -> (fwd ms,
# bwd ms, peak GiB). Different hardware: context for the same measurement here, not a target.
REFERENCE_PUBLISHED = {2048: (0.3402, 0.8208, 0.0914), 4096: (0.6385, 1.6529, 0.1847),
                       8192: (1.8703, 5.2663, 0.3772), 16384: (6.4977, 21.1941, 0.7856)}


def reference_shapes(seqs=(2048, 4096, 8192, 16384), batch: int = 2, heads: int = 12, head_dim: int = 64,
                     reps: int = 20) -> dict:
    """One attention layer's forward and backward timed as the reference's scripts/bench_kernels.py:30-59
    times them: bf16 q, k, v ~ N(0,1) (torch.manual_seed(0)) and a bf16 weight; the forward, a
    synchronize, then (out.to(bf16) * weight).sum().backward() and a synchronize, host clock around
    each half, 3 warm-ups and the mean of `reps`; peak memory is the allocator's high-water mark over
    the timed steps, inputs included."""
    import time

    rows = {}
    for seq in seqs:
        torch.manual_seed(0)
        q, k, v = (torch.randn(batch, heads, seq, head_dim, device="cuda", dtype=torch.bfloat16, requires_grad=True)
                   for _ in range(3))
        weight = torch.randn(batch, heads, seq, head_dim, device="cuda", dtype=torch.bfloat16)

        def step():
            out = kernels.selective_attention(q, k, v, dot_precision="bf16")
            torch.cuda.synchronize()
            mid = time.perf_counter()
            (out.to(weight.dtype) * weight).sum().backward()
            torch.cuda.synchronize()
            q.grad = k.grad = v.grad = None
            return mid

        for _ in range(3):
            step()
        torch.cuda.reset_peak_memory_stats()
        fwd = bwd = 0.0
        for _ in range(reps):
            torch.cuda.synchronize()
            start = time.perf_counter()
            mid = step()
            end = time.perf_counter()
            fwd += mid - start
            bwd += end - mid
        fwd_ms, bwd_ms = 1e3 * fwd / reps, 1e3 * bwd / reps
        row = {"fwd_ms": fwd_ms, "bwd_ms": bwd_ms, "total_ms": fwd_ms + bwd_ms,
               "peak_gib": torch.cuda.max_memory_allocated() / 2**30,
               "tflops": 7.0 * batch * heads * head_dim * seq * seq / ((fwd_ms + bwd_ms) * 1e-3) / 1e12}
        if seq in REFERENCE_PUBLISHED:
            rf, rb, rp = REFERENCE_PUBLISHED[seq]
            row["reference_published"] = {"fwd_ms": rf, "bwd_ms": rb, "total_ms": rf + rb, "peak_gib": rp}
        rows[str(seq)] = row
        del q, k, v, weight
        torch.cuda.empty_cache()
    return {"config": f"one layer fwd+bwd at the reference's published shapes: B={batch} H={heads} D={head_dim} bf16, "
                      f"timed as scripts/bench_kernels.py (host clock per half, {reps} reps)",
            "reference_source": "results/bench/layer_fwd_bwd_v2.json:26-93 (RTX PRO 6000 Blackwell; context only)",
            "by_seq": rows}


# Products each timed kernel computes (recomputation included), in units of one causal product over
# all heads (B H D T^2 FLOP): the forward QK^T and PV; the key-side backward QK^T, dO V^T, P^T dO,
# dz^T Q; the query-side backward QK^T, dO V^T, dz K.
KERNEL_PRODUCTS = {"forward": 2.0, "backward_kv": 4.0, "backward_dq": 3.0}
_KERNEL_IDS = {"forward": _lib.KERNEL_FORWARD, "backward_kv": _lib.KERNEL_BACKWARD,
               "backward_dq": _lib.KERNEL_BACKWARD_DQ, "selection": _lib.KERNEL_SELECTION}


def kernel_times(fn, calls: int, per_call: bool = False) -> dict:
    """Milliseconds of the library's main kernels over `calls` calls of fn(), from the HIP events the
    library records on each launch's own stream (sa_timing_*): the average per launch, or with
    per_call the summed time of each kernel per call of fn()."""
    torch.cuda.synchronize()
    _lib.timing_enable(True)
    for _ in range(calls):
        fn()
    torch.cuda.synchronize()
    res = {}
    for name, kid in _KERNEL_IDS.items():
        total, n = _lib.timing_read(kid)
        res[name] = total / calls if per_call else total / max(n, 1)
    _lib.timing_enable(False)
    return res


def decode_rate(t: int = 131072, batch: int = 1, heads: int = 16, head_dim: int = 64, steps: int = 50,
                warmup: int = 5) -> dict:
    """One cached decode step of one layer (the newest query of every head over t cached keys,
    bf16 cache, head 0 selecting): HBM bandwidth of the step against the 8 TB/s roof. Bytes: the K
    and V rows read once, the selection state read and written (fp32). `ms` is the whole call
    (host work of the wrapper included, which bounds small caches); `kernel_ms` the cache-reading
    kernel alone, from HIP events around it."""
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(6)
    k, v = (torch.randn(batch, heads, t, head_dim, device=dev, generator=g).bfloat16() for _ in range(2))
    q = torch.randn(batch, heads, head_dim, device=dev, generator=g).bfloat16()
    sel = torch.rand(batch, 1, t, device=dev, generator=g)

    def step():
        kernels.selective_attention_decode(q, k, v, sel)

    ms = _timed(step, steps, warmup)
    _lib.timing_enable(True)
    for _ in range(steps):
        step()
    kms, launches = _lib.timing_read(_lib.KERNEL_DECODE)
    _lib.timing_enable(False)
    kms /= max(launches, 1)
    nbytes = 2 * batch * heads * t * head_dim * 2 + 2 * batch * t * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"config": f"decode step, B={batch} H={heads} t={t} D={head_dim} bf16 cache, shared selection",
            "ms": ms, "bytes": nbytes, "gb_per_s": gbs, "frac_of_hbm_peak": gbs / 8000.0,
            "tokens_per_s": batch / (ms * 1e-3), "kernel_ms": kms,
            "kernel_gb_per_s": nbytes / (kms * 1e-3) / 1e9}


def copy_probe(mib: int = 1024, reps: int = 3) -> dict:
    """A plain device-to-device copy of `mib` MiB, `reps` times: the reference point that scales the
    FETCH_SIZE / WRITE_SIZE counters of rocprofv3 (each copy reads and writes exactly `mib` MiB)."""
    dev = torch.device("cuda")
    src = torch.ones(mib * 2**20 // 4, device=dev)
    dst = torch.empty_like(src)
    ms = _timed(lambda: dst.copy_(src), reps, 1)
    return {"config": f"copy of {mib} MiB", "ms": ms, "gb_per_s": 2 * mib * 2**20 / (ms * 1e-3) / 1e9}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("which", choices=["c3", "c4", "c5", "decode", "copy"])
    ap.add_argument("--geometry", default=None, choices=sorted(GEOMETRIES))
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--layers", type=int, default=24)
    ap.add_argument("--tokens", type=int, default=131072)
    ap.add_argument("--chunk", type=int, default=16384)
    a = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("needs a ROCm GPU", file=sys.stderr)
        return 2
    kw = {k: v for k, v in (("steps", a.steps), ("warmup", a.warmup)) if v is not None}
    if a.which == "c3":
        res = train_step_rate(a.geometry or "d768", layers=a.layers, **kw)
    elif a.which == "c4":
        res = prefill_rate(a.tokens, a.chunk, a.geometry or "d1024", a.layers,
                           **({"reps": a.steps} if a.steps else {}), **({"warmup": a.warmup} if a.warmup is not None else {}))
    elif a.which == "c5":
        res = perhead_rate(**kw)
    elif a.which == "decode":
        res = decode_rate(t=a.tokens, **kw)
    else:
        res = copy_probe()
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
