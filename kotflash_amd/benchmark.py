"""Interleaved benchmark of the HIP kernels against PyTorch SDPA on one device.

    python -m kotflash_amd.benchmark --seq 4096 --head-dim 128 --causal

Same command-line arguments and report fields as the reference's attention
benchmark (benchmarks/benchmark_attention.py:67-248):

- Every backend is warmed up (forward and training step) before anything is
  timed.
- Each of ``--repeats`` rounds then measures every backend once, in an order
  shuffled by a seeded RNG and recorded in the report. Figures are medians of
  the per-round medians.
- GPU timing uses HIP events around each call. The incremental peak of
  allocated memory is taken per measurement.
- Each backend's forward output is compared with SDPA on repeat-interleaved
  K/V.

Backends: ``pytorch_sdpa_native_gqa`` and ``pytorch_sdpa_expanded_kv`` (the
reference's baselines), ``hip`` (this build's kernels; the reference's
``triton`` slot) and ``auto``. A backend that cannot run on the device is
listed under ``backend_failures`` instead of being timed.
"""
from __future__ import annotations

import argparse
import json
import random
import statistics
import time
from typing import Callable, Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F

from .attention import attention


def _sync(device: torch.device) -> None:
    if device.type == "cuda":
        torch.cuda.synchronize(device)


def _measure(fn: Callable[[], None], iterations: int,
             device: torch.device) -> Tuple[float, Optional[int]]:
    """Median latency in ms of ``iterations`` calls, and the incremental peak
    of allocated device memory over them (None on the CPU)."""
    if device.type != "cuda":
        times = []
        for _ in range(iterations):
            t0 = time.perf_counter()
            fn()
            times.append((time.perf_counter() - t0) * 1e3)
        return statistics.median(times), None
    _sync(device)
    base = torch.cuda.memory_allocated(device)
    torch.cuda.reset_peak_memory_stats(device)
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(iterations)]
    for start, end in marks:
        start.record()
        fn()
        end.record()
    _sync(device)
    peak = max(0, torch.cuda.max_memory_allocated(device) - base)
    return statistics.median(s.elapsed_time(e) for s, e in marks), peak


def _summary(values: List[float]) -> dict:
    return {"median": statistics.median(values), "min": min(values), "max": max(values),
            "per_round": values}


def _environment(device: torch.device) -> dict:
    env = {"device": str(device), "torch": torch.__version__,
           "hip_runtime": getattr(torch.version, "hip", None)}
    if device.type == "cuda":
        props = torch.cuda.get_device_properties(device)
        env.update(gpu=torch.cuda.get_device_name(device),
                   arch=getattr(props, "gcnArchName", None),
                   compute_units=props.multi_processor_count,
                   memory_bytes=props.total_memory)
    else:
        env.update(gpu="CPU", threads=torch.get_num_threads())
    return env


def run(args: argparse.Namespace) -> dict:
    device = torch.device(args.device)
    dtype = torch.float16 if device.type == "cuda" else torch.float32
    sk = args.kv_seq or args.seq
    gen = torch.Generator().manual_seed(args.seed)

    def randn(*shape):
        return torch.randn(*shape, generator=gen).to(device=device, dtype=dtype).requires_grad_(True)

    q = randn(args.batch, args.q_heads, args.seq, args.head_dim)
    k = randn(args.batch, args.kv_heads, sk, args.head_dim)
    v = randn(args.batch, args.kv_heads, sk, args.head_dim)
    group = args.q_heads // args.kv_heads

    def expanded_sdpa():
        ke = k.repeat_interleave(group, dim=1) if group > 1 else k
        ve = v.repeat_interleave(group, dim=1) if group > 1 else v
        return F.scaled_dot_product_attention(q, ke, ve, is_causal=args.causal)

    backends: Dict[str, Callable[[], torch.Tensor]] = {
        "pytorch_sdpa_native_gqa": lambda: attention(q, k, v, causal=args.causal, backend="sdpa"),
        "pytorch_sdpa_expanded_kv": expanded_sdpa,
        "hip": lambda: attention(q, k, v, causal=args.causal, backend="hip"),
        "auto": lambda: attention(q, k, v, causal=args.causal, backend="auto"),
    }

    def forward(fn):
        def call():
            with torch.no_grad():
                fn()
        return call

    def train(fn):
        def call():
            q.grad = k.grad = v.grad = None
            fn().float().square().mean().backward()
        return call

    train_iters = max(5, args.iterations // 4)
    train_warmup = max(2, args.warmup // 4)
    ready: Dict[str, Tuple[Callable, Callable]] = {}
    failures: Dict[str, str] = {}
    for name, fn in backends.items():
        try:
            f, t = forward(fn), train(fn)
            for _ in range(args.warmup):
                f()
            for _ in range(train_warmup):
                t()
            _sync(device)
            ready[name] = (f, t)
        except Exception as exc:  # recorded, not fatal: e.g. hip on a CPU
            failures[name] = f"{type(exc).__name__}: {exc}"

    with torch.no_grad():
        reference = expanded_sdpa().float()
    samples = {n: {"fwd": [], "train": [], "fwd_peak": [], "train_peak": [], "err": None}
               for n in ready}
    rng = random.Random(args.seed)
    orders = []
    for _ in range(args.repeats):
        order = list(ready)
        rng.shuffle(order)
        orders.append(order)
        for name in order:
            f, t = ready[name]
            with torch.no_grad():
                err = (backends[name]().float() - reference).abs().max().item()
            f_ms, f_peak = _measure(f, args.iterations, device)
            q.grad = k.grad = v.grad = None
            t_ms, t_peak = _measure(t, train_iters, device)
            s = samples[name]
            s["fwd"].append(f_ms)
            s["train"].append(t_ms)
            if f_peak is not None:
                s["fwd_peak"].append(f_peak)
                s["train_peak"].append(t_peak)
            s["err"] = err

    report = {
        "environment": _environment(device),
        "shape": {"B": args.batch, "Hq": args.q_heads, "Hkv": args.kv_heads, "Sq": args.seq,
                  "Sk": sk, "D": args.head_dim},
        "dtype": str(dtype),
        "causal": args.causal,
        "warmup": args.warmup,
        "iterations_per_round": args.iterations,
        "backward_iterations_per_round": train_iters,
        "repeats": args.repeats,
        "seed": args.seed,
        "measurement_order_by_round": orders,
        "comparison_note": ("every backend warmed before timing; per-round order shuffled with a "
                            "fixed seed; figures are medians of per-round medians; expanded-KV "
                            "includes the repeat_interleave cost"),
    }
    for name, s in samples.items():
        report[name] = {
            "forward_ms": _summary(s["fwd"]),
            "forward_backward_ms": _summary(s["train"]),
            "forward_incremental_peak_allocated_bytes":
                int(statistics.median(s["fwd_peak"])) if s["fwd_peak"] else None,
            "forward_backward_incremental_peak_allocated_bytes":
                int(statistics.median(s["train_peak"])) if s["train_peak"] else None,
            "max_abs_error_vs_expanded_sdpa": s["err"],
        }
    if failures:
        report["backend_failures"] = failures
    for cand in ("hip", "auto"):
        for base in ("pytorch_sdpa_native_gqa", "pytorch_sdpa_expanded_kv"):
            for metric, key in (("forward", "forward_ms"), ("forward_backward", "forward_backward_ms")):
                c = report.get(cand, {}).get(key)
                b = report.get(base, {}).get(key)
                if c and b and c["median"] > 0:
                    report[f"{cand}_{metric}_speedup_vs_{base}"] = b["median"] / c["median"]
    return report


def parse_args(argv: Optional[List[str]] = None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--device", default="cuda")
    p.add_argument("--batch", type=int, default=2)
    p.add_argument("--q-heads", type=int, default=16)
    p.add_argument("--kv-heads", type=int, default=4)
    p.add_argument("--seq", type=int, default=1024)
    p.add_argument("--kv-seq", type=int, default=None)
    p.add_argument("--head-dim", type=int, default=64)
    p.add_argument("--causal", action="store_true")
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--iterations", type=int, default=50)
    p.add_argument("--repeats", type=int, default=5)
    p.add_argument("--seed", type=int, default=1337)
    args = p.parse_args(argv)
    if min(args.batch, args.q_heads, args.kv_heads, args.seq, args.head_dim) <= 0:
        p.error("batch, head counts, sequence length and head dimension must be positive")
    if args.q_heads % args.kv_heads:
        p.error("--q-heads must be divisible by --kv-heads")
    if args.kv_seq is not None and args.kv_seq <= 0:
        p.error("--kv-seq must be positive")
    if args.warmup < 0 or args.iterations <= 0 or args.repeats < 3:
        p.error("warmup must be non-negative, iterations positive and repeats at least 3")
    if args.device.startswith("cuda") and not torch.cuda.is_available():
        p.error("a GPU was requested but torch.cuda.is_available() is False")
    return args


def main(argv: Optional[List[str]] = None) -> None:
    print(json.dumps(run(parse_args(argv)), indent=2, default=str))


if __name__ == "__main__":
    main()
