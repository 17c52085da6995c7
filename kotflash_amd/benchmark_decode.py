"""One-token GQA decode benchmark: attention alone and append + attention.

    python -m kotflash_amd.benchmark_decode --batch 2 --q-heads 8 --kv-heads 2 --head-dim 64 --kv-seq 16384

The same arguments and report fields as the reference's decode benchmark
(benchmarks/benchmark_decode.py:34-321), on this build's backends:

- ``hip`` (the reference's ``triton`` slot) and ``auto`` through
  ``attention``, on the visible K/V and, for append + attention, after
  ``append_kv_cache`` (a ``torch.cat`` of the whole history, as the
  reference's legacy path);
- ``pytorch_expanded_sdpa``, SDPA on K/V expanded to Hq heads (the baseline
  every speedup is quoted against);
- ``preallocated_hip_separate_append`` (torch-copy append, then the HIP
  decode reading the strided prefix view), ``preallocated_auto`` (the
  ``--append-backend`` choice) and ``preallocated_fused_append`` (one split
  kernel that also writes the new token, then the merge).

Every candidate's output, attention alone and append + attention, is
checked against the expanded-SDPA output first (rtol = atol = 8e-3, the
reference's figure; the reference checks the attention-only output). Per
candidate and metric the report gives GPU-event and synchronized wall-clock medians,
minima and maxima over ``--repeats`` repeats of ``--iterations`` calls, the
incremental peak of allocated memory, and speedups against the baseline.
With ``--device cpu`` only the SDPA candidates run (the HIP ones are listed
under ``backend_failures``), so the report's structure can be checked
without a GPU.
"""
from __future__ import annotations

import argparse
import json
import statistics
import time
from pathlib import Path
from typing import Any, Callable, List, Optional

import torch
import torch.nn.functional as F

from .attention import attention
from .benchmark import _environment, _sync
from .cache import PreallocatedKVCache, append_kv_cache

APPEND_BACKENDS = ("auto", "torch", "hip", "cuda", "fused")


def measure(fn: Callable[[], Any], *, warmup: int, iterations: int, repeats: int,
            device: torch.device) -> dict:
    """GPU-event and wall-clock ms per call over ``repeats`` repeats of
    ``iterations`` back-to-back calls, plus the incremental peak of allocated
    memory (None on the CPU)."""
    cuda = device.type == "cuda"
    with torch.inference_mode():
        for _ in range(warmup):
            fn()
        _sync(device)
        if cuda:
            base = torch.cuda.memory_allocated(device)
            torch.cuda.reset_peak_memory_stats(device)
        gpu: List[float] = []
        wall: List[float] = []
        for _ in range(repeats):
            if cuda:
                start, end = (torch.cuda.Event(enable_timing=True) for _ in range(2))
            t0 = time.perf_counter()
            if cuda:
                start.record()
            for _ in range(iterations):
                fn()
            if cuda:
                end.record()
            _sync(device)
            wall.append((time.perf_counter() - t0) * 1e3 / iterations)
            if cuda:
                gpu.append(start.elapsed_time(end) / iterations)
        peak = max(0, torch.cuda.max_memory_allocated(device) - base) if cuda else None
    gpu = gpu or wall  # on the CPU the device time is the wall time
    return {
        "gpu_median_ms": statistics.median(gpu), "gpu_min_ms": min(gpu), "gpu_max_ms": max(gpu),
        "gpu_per_repeat_ms": gpu,
        "wall_median_ms": statistics.median(wall), "wall_min_ms": min(wall),
        "wall_max_ms": max(wall), "wall_per_repeat_ms": wall,
        "incremental_peak_allocated_bytes": None if peak is None else int(peak),
    }


def run(args: argparse.Namespace) -> dict:
    device = torch.device(args.device)
    dtype = torch.float16 if device.type == "cuda" else torch.float32
    gen = torch.Generator().manual_seed(args.seed)

    def randn(*shape):
        return torch.randn(*shape, generator=gen).to(device=device, dtype=dtype)

    b, hq, hkv, d, sk = args.batch, args.q_heads, args.kv_heads, args.head_dim, args.kv_seq
    q = randn(b, hq, 1, d)
    past_k, past_v = randn(b, hkv, sk - 1, d), randn(b, hkv, sk - 1, d)
    new_k, new_v = randn(b, hkv, 1, d), randn(b, hkv, 1, d)
    visible_k, visible_v = append_kv_cache(past_k, past_v, new_k, new_v)
    group = hq // hkv
    # Unused capacity after the visible prefix, so the cache views are strided.
    capacity = max(2 * sk, sk + 16)
    prefilled = PreallocatedKVCache(b, hkv, capacity, d, device=device, dtype=dtype)
    prefilled.append(visible_k, visible_v, backend="torch")
    decode_cache = PreallocatedKVCache(b, hkv, capacity, d, device=device, dtype=dtype)
    decode_cache.append(past_k, past_v, backend="torch")

    def expanded(k, v):
        return F.scaled_dot_product_attention(q, k.repeat_interleave(group, 1),
                                              v.repeat_interleave(group, 1))

    def legacy(backend):
        def attend():
            return attention(q, visible_k, visible_v, causal=False, backend=backend)

        def decode():
            k, v = append_kv_cache(past_k, past_v, new_k, new_v)
            return attention(q, k, v, causal=False, backend=backend)
        return attend, decode

    def preallocated(attend_backend, append_backend):
        def attend():
            return prefilled.attend(q, backend=attend_backend)

        def decode():
            # Only the logical length is reset: the same slot is rewritten on
            # every call and no history is copied.
            decode_cache.length = sk - 1
            return decode_cache.append_and_attend(q, new_k, new_v, append_backend=append_backend,
                                                  attention_backend=attend_backend)
        return attend, decode

    candidates = {
        "hip": legacy("hip"),
        "auto": legacy("auto"),
        "pytorch_expanded_sdpa": (lambda: expanded(visible_k, visible_v),
                                  lambda: expanded(*append_kv_cache(past_k, past_v, new_k, new_v))),
        "preallocated_hip_separate_append": preallocated("hip", "torch"),
        "preallocated_auto": preallocated("auto", args.append_backend),
        "preallocated_fused_append": preallocated("hip", "fused"),
    }
    failures = {}
    correctness = {}
    with torch.inference_mode():
        reference = expanded(visible_k, visible_v)
        for name, fns in list(candidates.items()):
            checks = {}
            for metric, fn in zip(("attention_only", "append_plus_attention"), fns):
                try:
                    out = fn()
                    _sync(device)
                except (RuntimeError, ValueError, TypeError) as exc:
                    failures[name] = f"{type(exc).__name__}: {exc}"
                    break
                err = float((out.float() - reference.float()).abs().max())
                finite = bool(torch.isfinite(out).all())
                close = bool(torch.allclose(out.float(), reference.float(), rtol=8e-3, atol=8e-3))
                checks[metric] = {"max_abs_error_vs_expanded_sdpa": err, "finite": finite,
                                  "within_tolerance": close}
                if not (finite and close):
                    raise RuntimeError(f"{name} ({metric}) failed the expanded-SDPA correctness "
                                       f"check: finite={finite}, max_abs_error={err}")
            if name in failures:
                del candidates[name]
            else:
                correctness[name] = checks

    timing = dict(warmup=args.warmup, iterations=args.iterations, repeats=args.repeats,
                  device=device)
    report = {
        "benchmark": "one-token GQA decode; attention-only and append+attention",
        "environment": _environment(device),
        "shape": {"batch": b, "q_heads": hq, "kv_heads": hkv, "query_length": 1,
                  "visible_kv_length": sk, "head_dim": d},
        "dtype": str(dtype),
        "seed": args.seed,
        "warmup": args.warmup,
        "iterations_per_repeat": args.iterations,
        "repeats": args.repeats,
        "append_backend": args.append_backend,
        "preallocated_cache_capacity": capacity,
        "preallocated_cache_layout": "strided prefix view; unused capacity follows the visible prefix",
        "cache_append_only": measure(lambda: append_kv_cache(past_k, past_v, new_k, new_v),
                                     **timing),
        "correctness": correctness,
        "backend_failures": failures,
        "results": {},
        "interpretation": (
            "batch_tokens_per_second is throughput for one decode position per batch "
            "entry, from the wall-clock median; it excludes projections, MLP, sampling "
            "and scheduling. The legacy append_plus_attention variants include torch.cat "
            "of the history; preallocated variants write into fixed storage, and "
            "fused_append stores the new token from inside the split-KV kernel. GPU event "
            "time and synchronized wall-clock time are reported separately."),
    }
    for name, (attend, decode) in candidates.items():
        a = measure(attend, **timing)
        dec = measure(decode, **timing)
        dec["batch_tokens_per_second"] = b * 1000.0 / dec["wall_median_ms"]
        report["results"][name] = {"attention_only": a, "append_plus_attention": dec}
    base = report["results"]["pytorch_expanded_sdpa"]
    for values in report["results"].values():
        for metric in ("attention_only", "append_plus_attention"):
            for clock in ("gpu", "wall"):
                values[metric][f"{clock}_speedup_vs_expanded_sdpa"] = (
                    base[metric][f"{clock}_median_ms"] / values[metric][f"{clock}_median_ms"])
    return report


def parse_args(argv: Optional[List[str]] = None) -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__.split("\n", 1)[0])
    ap.add_argument("--batch", type=int, default=2)
    ap.add_argument("--q-heads", type=int, default=8)
    ap.add_argument("--kv-heads", type=int, default=2)
    ap.add_argument("--head-dim", type=int, default=64)
    ap.add_argument("--kv-seq", type=int, default=2048)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--iterations", type=int, default=50)
    ap.add_argument("--repeats", type=int, default=5)
    ap.add_argument("--append-backend", choices=APPEND_BACKENDS, default="auto",
                    help="append implementation of the preallocated_auto candidate")
    ap.add_argument("--seed", type=int, default=1337)
    ap.add_argument("--device", default="cuda")
    ap.add_argument("--output", type=Path, default=None)
    args = ap.parse_args(argv)
    if min(args.batch, args.q_heads, args.kv_heads, args.head_dim, args.kv_seq) <= 0:
        ap.error("all tensor dimensions must be positive")
    if args.q_heads % args.kv_heads:
        ap.error("--q-heads must be divisible by --kv-heads")
    if args.head_dim % 8 or not 8 <= args.head_dim <= 128:
        ap.error("the split-KV decode needs --head-dim a multiple of 8 in [8, 128]")
    if args.kv_seq < 1024:
        ap.error("the split-KV decode benchmark needs --kv-seq >= 1024")
    if args.warmup < 1 or args.iterations < 1 or args.repeats < 3:
        ap.error("use warmup >= 1, iterations >= 1 and repeats >= 3")
    if args.device.startswith("cuda") and not torch.cuda.is_available():
        ap.error("no GPU visible; pass --device cpu to check the report on the CPU")
    return args


def main(argv: Optional[List[str]] = None) -> None:
    args = parse_args(argv)
    report = run(args)
    text = json.dumps(report, indent=2, default=str)
    print(text)
    if args.output is not None:
        args.output.parent.mkdir(parents=True, exist_ok=True)
        args.output.write_text(text + "\n", encoding="utf-8")


if __name__ == "__main__":
    main()
