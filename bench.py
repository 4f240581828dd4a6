"""Benchmark of the Selective Attention operator on one MI355X (BASELINE config C2 and the rest).

One step = one fused forward + backward of the operator through the reference's API
(`selective_attention(q, k, v)` then the gradients of q, k, v for an upstream gradient dO) at
B=1, H=16, T=16384, D=64 in bf16, inputs already resident in HBM. The step includes everything
the autograd op launches: the selection scan, the forward, the backward's transposes / row
statistics, the two backward kernels and the gradient epilogue.

Printed (one JSON line): TFLOP/s under the FlashAttention convention (forward 2*B*H*D*T^2,
forward + backward 7*B*H*D*T^2, causal pairs counted as T^2/2), the roofline of the dominant kernel
(the longest of the forward, key-side backward and query-side backward kernels: the products it
computes / its average HIP-event duration inside the timed region, against the 2.5 PFLOP/s dense
bf16 MFMA peak), and CPU baselines: the fp32 listing (the test oracle) timed on this host for a
bounded sample of the C2 workload, and at C1's own shape.

The same line carries BASELINE's other configurations (selective_attention/harness.py):
  train   C3, full training steps of the 24-layer decoder at 1 x 16384 tokens, both geometries
          (the reference's 209M d768 / 12 heads, and BASELINE's literal d1024 / 16 heads)
  c4      C4, the 131072-token prefill in 8 chunks of 16384 through 24 d1024 layers
  c5      C5, per-head selection fwd+bwd at B=2 H=16 T=32768 D=64 with its dominant kernel's roofline
  reference_shapes  one layer's fwd and bwd at the reference's own published shapes (B=2 H=12 D=64,
          T = 2K ... 16K), timed as its scripts/bench_kernels.py does, beside its published figures
          (other hardware: context, not a target)

    python bench.py [--steps K] [--warmup W] [--no-cpu-baseline] [--no-train] [--no-configs] [--no-ref-shapes]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "selective-attention-study_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

B, H, T, D = 1, 16, 16384, 64
PEAK_BF16_TFLOPS = 2500.0          # MI355X dense bf16 MFMA, published
UNIT = B * H * D * T * T           # one causal product (T^2/2 pairs x D x 2 FLOP) over all heads
STEP_FLOP = 7.0 * UNIT             # fwd 2 products + bwd 5 (FlashAttention convention) = 1.9241e12
# Products each timed kernel computes (recomputation included): the forward QK^T and PV; the
# key-side backward QK^T, dO V^T, P^T dO, dz^T Q; the query-side backward QK^T, dO V^T, dz K.
KERNEL_FLOP = {"forward": 2.0 * UNIT, "backward_kv": 4.0 * UNIT, "backward_dq": 3.0 * UNIT}
# HBM bytes per launch of each kernel at this workload, measured with rocprofv3's FETCH_SIZE and
# WRITE_SIZE counters (one pass each) and scaled by a 1 GiB copy's readings (FETCH x 2.0, WRITE x
# 1.0): profiles/c2_attention_kernels_traffic.md. The counters need the profiler, so bench.py
# reports the committed measurement, labelled with the hash of the kernel sources it was taken on
# (PROFILED_SOURCES): the line says whether the sources it runs are still those.
MEASURED_TRAFFIC_BYTES = {"forward": (2.0 * 460_700 + 67_588) * 1024,
                          "backward_kv": (2.0 * 330_872 + 391_687) * 1024,
                          "backward_dq": (2.0 * 352_457 + 96_256) * 1024}
# C4 (131072-token prefill, 8 chunks): the forward kernel's HBM bytes per launch (mean over the
# chunks, FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0) and MFMA busy fraction, measured with rocprofv3:
# profiles/c4_prefill_kernels.md. The run's own per-launch time turns the bytes into a rate.
MEASURED_C4 = {"hbm_bytes_per_launch": (2.0 * 3_288_204 + 67_584) * 1024, "mfma_busy": 0.35}
# sha256 (first 16 hex digits) of csrc/sa_kernels.h when the figures above were profiled
PROFILED_SOURCES = "686b814c501d5591"
KERNEL_SOURCE = os.path.join(ROOT, "selective-attention-study_amd", "csrc", "sa_kernels.h")


def _profiled_label() -> dict:
    """Where the committed counter figures come from, and whether this run's kernels are the ones
    they were taken on (the kernel source's hash against the one recorded with them)."""
    import hashlib

    try:
        with open(KERNEL_SOURCE, "rb") as f:
            now = hashlib.sha256(f.read()).hexdigest()[:16]
    except OSError:
        now = None
    return {"profiled_sources_sha16": PROFILED_SOURCES, "current_sources_sha16": now,
            "current": now == PROFILED_SOURCES}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(budget_s: float = 20.0) -> dict:
    """The fp32 listing (oracle/sa_oracle.py) forward + autograd backward on the host CPU, on the C2
    parity slice B=1, H=16, T=2048, D=64: one warm-up, then repetitions until about budget_s."""

    import torch

    from oracle import sa_oracle

    t = 2048
    g = torch.Generator().manual_seed(0)
    q, k, v, do = (torch.randn(B, H, t, D, generator=g) for _ in range(4))
    q.requires_grad_(True), k.requires_grad_(True), v.requires_grad_(True)

    def run():
        out = sa_oracle.attention(q, k, v)
        torch.autograd.grad(out, (q, k, v), do)

    med, reps = _median_time(run, budget_s, 3)
    flop = 7.0 * B * H * D * t * t
    return {
        "value": flop / med / 1e12,
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"fp32 listing (oracle/sa_oracle.py, torch on CPU) fwd+bwd at B=1 H=16 T=2048 D=64, "
                   f"median of {reps} reps = {med * 1e3:.0f} ms; 7*B*H*D*T^2 FLOP; "
                   f"{len(os.sched_getaffinity(0))} cores visible, CPU {_cpu_model()}"),
    }


def cpu_c1(budget_s: float = 8.0) -> dict:
    """C1 as BASELINE states it: the fp32 listing forward on the host CPU at B=1, H=4, T=512, D=64,
    q, k, v ~ N(0,1) drawn in that order from one seed; median of >= 10 reps after 2 warm-ups."""

    import torch

    from oracle import sa_oracle

    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, 4, 512, 64, generator=g) for _ in range(3))
    with torch.no_grad():
        med, reps = _median_time(lambda: sa_oracle.attention(q, k, v), budget_s, 10, warmup=2)
    flop = 2.0 * 1 * 4 * 64 * 512 * 512
    return {"config": "C1: fp32 listing forward on CPU, B=1 H=4 T=512 D=64 (oracle/sa_oracle.py)",
            "ms": med * 1e3, "reps": reps, "gflops": flop / med / 1e9, "cores": torch.get_num_threads(),
            "cpu": _cpu_model()}


def _median_time(fn, budget_s: float, min_reps: int, warmup: int = 1) -> tuple[float, int]:
    for _ in range(warmup):
        fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < min_reps:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def _progress(msg: str) -> None:
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def _rounded(d: dict) -> dict:
    return {k_: (round(v_, 4) if isinstance(v_, float) else (_rounded(v_) if isinstance(v_, dict) else v_))
            for k_, v_ in d.items()}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-train", action="store_true", help="skip the 24-layer training-step rates (C3)")
    ap.add_argument("--no-configs", action="store_true", help="skip the C4 prefill and C5 per-head rates")
    ap.add_argument("--no-ref-shapes", action="store_true",
                    help="skip the one-layer timings at the reference's published shapes (B=2 H=12)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: the operator runs on a single MI355X "
              "(sharding across GPUs is a design here, not a code path)", file=sys.stderr)
        return 2

    import torch

    from selective_attention import _lib, kernels

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    if not kernels.HAS_HIP:
        _lib.load()   # raises with the reason
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v = (torch.randn(B, H, T, D, device=dev, generator=g).bfloat16().requires_grad_(True) for _ in range(3))
    do = torch.randn(B, H, T, D, device=dev, generator=g)

    def step():
        out = kernels.selective_attention(q, k, v)
        return torch.autograd.grad(out, (q, k, v), do)

    torch.cuda.reset_peak_memory_stats()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    _lib.timing_enable(True)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        grads = step()
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / args.steps
    peak_gib = torch.cuda.max_memory_allocated() / 2**30
    per_kernel = {}
    for name, kid in (("forward", _lib.KERNEL_FORWARD), ("backward_kv", _lib.KERNEL_BACKWARD),
                      ("backward_dq", _lib.KERNEL_BACKWARD_DQ), ("selection", _lib.KERNEL_SELECTION)):
        total, n = _lib.timing_read(kid)
        per_kernel[name] = total / max(n, 1)
    _lib.timing_enable(False)
    assert all(torch.isfinite(gr).all().item() for gr in grads)

    tflops = STEP_FLOP / (ms * 1e-3) / 1e12
    dominant = max(KERNEL_FLOP, key=lambda name: per_kernel[name])
    achieved = KERNEL_FLOP[dominant] / (per_kernel[dominant] * 1e-3) / 1e12
    record = {
        "metric": "fused fwd+bwd TFLOP/s & MFMA util at T=16K H=16 D=64 bf16; train tok/s",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: q, k, v, dO ~ N(0,1), fixed seed",
        "config": {"workload": "C2: selective attention fused fwd+bwd, B=1 H=16 T=16384 D=64, exempt=1 (BOS)",
                   "flop_per_step": STEP_FLOP, "flop_convention": "7*B*H*D*T^2 (fwd 2, bwd 5; causal T^2/2)"},
        "frac_of_peak": round(tflops / PEAK_BF16_TFLOPS, 4),
        "kernel_ms": {k_: round(v_, 4) for k_, v_ in per_kernel.items()},
        "peak_mem_gib": round(peak_gib, 4),
        "roofline": {"bound": "mfma",
                     "kernel": f"{dominant} ({KERNEL_FLOP[dominant] / UNIT:.0f}*B*H*D*T^2 FLOP per launch)",
                     "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": MEASURED_TRAFFIC_BYTES[dominant], "traffic_unit": "bytes per launch (rocprofv3)",
                     "traffic_source": dict(_profiled_label(), file="profiles/c2_attention_kernels_traffic.md")},
    }
    del q, k, v, do, grads
    torch.cuda.empty_cache()
    _progress(f"C2 {ms:.3f} ms/step")
    from selective_attention import harness

    if not args.no_train:
        # the metric's "train tok/s": C3 at the reference's 209M geometry (d768, 12 heads x 64) and at
        # BASELINE's literal one (d1024, 16 heads x 64), 24 layers, 1 x 16384 tokens
        record["train"] = {}
        for geometry in ("d768", "d1024"):
            tr = harness.train_step_rate(geometry, steps=10, warmup=3)
            record["train"][geometry] = _rounded(tr)
            torch.cuda.empty_cache()
            _progress(f"C3 {geometry} {tr['tokens_per_s']:.0f} tok/s")
        record["train_tok_s"] = round(record["train"]["d768"]["tokens_per_s"], 1)
    if not args.no_configs:
        c4 = harness.prefill_rate(reps=2, warmup=1)
        c4["counters"] = {"source": dict(_profiled_label(), file="profiles/c4_prefill_kernels.md (rocprofv3 --pmc)"),
                          "mfma_busy": MEASURED_C4["mfma_busy"],
                          "hbm_bytes_per_launch": MEASURED_C4["hbm_bytes_per_launch"],
                          "hbm_tb_s": MEASURED_C4["hbm_bytes_per_launch"] / (c4["per_layer_chunk_forward_ms"] * 1e9),
                          "hbm_frac_of_peak": MEASURED_C4["hbm_bytes_per_launch"]
                          / (c4["per_layer_chunk_forward_ms"] * 1e-3) / 8e12}
        record["c4"] = _rounded(c4)
        torch.cuda.empty_cache()
        _progress(f"C4 {record['c4']['tokens_per_s']:.0f} tok/s")
        record["c5"] = _rounded(harness.perhead_rate(steps=5, warmup=2))
        torch.cuda.empty_cache()
        _progress(f"C5 {record['c5']['ms_per_step']:.2f} ms/step")
    if not args.no_ref_shapes:
        record["reference_shapes"] = _rounded(harness.reference_shapes())
        torch.cuda.empty_cache()
        _progress("reference shapes " + ", ".join(f"T={t_}: {r_['total_ms']:.2f} ms"
                                                  for t_, r_ in record["reference_shapes"]["by_seq"].items()))
    if not args.no_cpu_baseline:
        record["cpu_baseline"] = cpu_baseline()
        record["cpu_c1"] = _rounded(cpu_c1())
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
